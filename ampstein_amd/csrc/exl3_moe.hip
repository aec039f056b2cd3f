// Fused decode-shaped MoE for gfx950 (exl3_moe_coop semantics, quant/exl3_moe_coop_kernel.cuh,
// quant/exl3_moe_coop.cu): every (token, expert) slot through gate/up, activation and down, with
// per-expert bit widths (mixed K) or one uniform width.  Three stages:
//
//   route   block 0 sorts the active slots by (local expert, slot) and cuts runs of at most 8
//           slots of one expert into the caller's run table (exl3_moe_coop_kernel.cuh:273-356,
//           same layout); every wave rotates one 128-chunk of one slot's x row (zero-padded to
//           Hi, * suh in fp32, Hadamard, fp16) for gate and up; tokens without an active slot get
//           their output row here (shared-expert term or zeros).
//   A       one workgroup per (run, 128-column chunk, projection, k-split): the run's slots are
//           the rows of one multi-row GEMV over the expert's trellis (x in LDS as (x, x) pairs,
//           the decode of the dense GEMV); the last arrival of a (slot, chunk) sums the split
//           partials, rotates, * svh, + bias, applies the activation, * down suh, rotates and
//           stores the down input (:803-845).
//   B       the same GEMV over the down trellis; the last arrival of a (token, chunk) rotates
//           each active slot's sum * svh (+ bias), weights it by its routing weight, sums the
//           slots in the reference's fixed order (:917-999), adds the shared expert and stores.
// A and B each launch once per run size class: single-slot runs with the one-row body (126
// VGPRs, 4 waves per SIMD), larger runs with the eight-row body.  A token's slots can sit in
// both classes; its down hand-off counter then collects arrivals from both launches.
//
// Hand-offs: counters (one 128-byte line each) in the library workspace; chunk c runs on XCD
// c % 8 when the chunk counts allow, so the hand-off is an L2-local atomic, else device scope.
// Compiled once per codebook (EXL3_MOE_CB); the bit width is a per-workgroup switch.
#include "exl3_common.cuh"
#include "exl3_gemv_core.cuh"
#include "exl3_kernels.h"
#include "exl3_xcd.cuh"

#ifndef EXL3_MOE_CB
#define EXL3_MOE_CB 0
#endif
constexpr int EXL3_MOE_PF1 = 4;  // k-slices in flight per wave, single-row body, K <= 4

using namespace exl3;

namespace {

constexpr int NT = 256;          // threads per workgroup
constexpr int NW = NT / 64;      // waves
constexpr int ROWS = 8;          // slots per run (exl3_moe_coop_kernel.cuh:37)
constexpr int SBMAX = EXL3_MOE_SBMAX; // k-slices per workgroup (LDS: ROWS x SBMAX x 16 x-pairs)
constexpr int WKR = 16;          // slot-sum partition of the down epilogue (the reference's 16 warps)

struct SlotInfo
{
    int row;
    int local;
    float w;
    bool active;
};

// exl3_moe_coop_kernel.cuh:250-267
__device__ __forceinline__ SlotInfo slot_info(const MoeArgs& a, int s)
{
    SlotInfo si;
    si.row = s / a.topk;
    int64_t e = *to_global(a.sel + s);
    si.w = (float) as_h(*to_global(a.rw + s));
    bool ok = si.w != 0.0f;
    if (a.min_expert >= 0)
    {
        ok = ok && e >= a.min_expert && e < a.max_expert;
        e -= a.min_expert;
    }
    si.local = ok ? (int) e : 0;
    si.active = ok;
    return si;
}

__device__ __forceinline__ int token_active_slots(const MoeArgs& a, int row)
{
    int n = 0;
    for (int k = 0; k < a.topk; ++k) n += slot_info(a, row * a.topk + k).active ? 1 : 0;
    return n;
}

template <typename T>
__device__ __forceinline__ const T* tab(const uint64_t* table, int i) { return (const T*) *to_global(table + i); }

__device__ __forceinline__ float h2f(const uint16_t* p, int i) { return (float) as_h(*to_global(p + i)); }

// ---- activations (fp32; exl3_moe_coop_kernel.cuh:91-128).  GELU is the tanh approximation of
// Hendrycks & Gimpel with its published constants.
__device__ __forceinline__ float act_silu(float x) { return x / (1.0f + __expf(-x)); }
__device__ __forceinline__ float act_gelu(float x)
{
    const float c = 0.797884560803f;        // sqrt(2 / pi)
    return 0.5f * x * (1.0f + tanhf(c * (x + 0.044715f * x * x * x)));
}
__device__ __forceinline__ float act_relu2(float x) { x = fmaxf(0.0f, x); return x * x; }
__device__ __forceinline__ float act_oai(float g, float u, float limit)
{
    if (limit != 0.0f)
    {
        g = fminf(g, limit);
        u = fminf(fmaxf(u, -limit), limit);
    }
    const float glu = g * (1.0f / (1.0f + __expf(-1.702f * g)));
    return (u + 1.0f) * glu;
}
__device__ __forceinline__ float act_gate(int act, bool gated, float g, float u, float limit)
{
    if (act == 3) return act_oai(g, u, limit);
    float x;
    if (!gated) x = fmaxf(0.0f, u);
    else if (act == 0) x = act_silu(g);
    else if (act == 1) x = act_gelu(g);
    else x = act_relu2(g);
    if (limit != 0.0f)
    {
        u = fminf(fmaxf(u, -limit), limit);
        x = fminf(x, limit);
    }
    return x * u;
}

// ---- wave-level row chunk helpers: lane l holds columns 2l, 2l + 1 of a 128-chunk

__device__ __forceinline__ float wave_sum(float v, int lane)
{
    v += xor_partner<1>(v, lane);
    v += xor_partner<2>(v, lane);
    v += xor_partner<4>(v, lane);
    v += xor_partner<8>(v, lane);
    v += xor_partner<16>(v, lane);
    v += xor_partner<32>(v, lane);
    return v;
}

// sigmoid(x_row . sh_gate_w), fp32, by one wave
__device__ __forceinline__ float shared_gate(const MoeArgs& a, int row, int lane)
{
    const uint16_t* xr = a.x + (size_t) row * a.x_stride;
    float dot = 0.0f;
    for (int i = 2 * lane; i < a.H; i += 128)
    {
        dot += h2f(xr, i) * h2f(a.sh_gate_w, i);
        if (i + 1 < a.H) dot += h2f(xr, i + 1) * h2f(a.sh_gate_w, i + 1);
    }
    dot = wave_sum(dot, lane);
    return 1.0f / (1.0f + __expf(-dot));
}

// Token without an active slot: its output chunk is the shared-expert term or zeros (:605-643)
__device__ __forceinline__ void write_empty_row_chunk(const MoeArgs& a, int row, int chunk, int lane)
{
    const int col = chunk * 128 + 2 * lane;
    float o0 = 0.0f, o1 = 0.0f;
    if (a.sh_out)
    {
        const float gv = a.sh_gate_w ? shared_gate(a, row, lane) : 1.0f;
        const float* sh = a.sh_out + (size_t) row * a.H + col;
        if (col < a.H) o0 = gv * *to_global(sh);
        if (col + 1 < a.H) o1 = gv * *to_global(sh + 1);
    }
    float* dst = a.out + (size_t) row * a.out_stride + col;
    if (col < a.H_out) *to_global_w(dst) = o0;
    if (col + 1 < a.H_out) *to_global_w(dst + 1) = o1;
}

// Input rotation of one 128-chunk of a slot's x row: zero-padded to Hi, * suh (fp32), Hadamard,
// fp16 (:646-663)
__device__ __forceinline__ void rotate_chunk(const MoeArgs& a, int row, const uint16_t* suh, int c, uint16_t* dst, int lane)
{
    const int col = c * 128 + 2 * lane;
    const uint16_t* xr = a.x + (size_t) row * a.x_stride;
    float v0 = col < a.H ? h2f(xr, col) : 0.0f;
    float v1 = col + 1 < a.H ? h2f(xr, col + 1) : 0.0f;
    v0 *= h2f(suh, col);
    v1 *= h2f(suh, col + 1);
    fwht128_wave(v0, v1, lane);
    const f16x2 o = { (f16) (v0 * EXL3_HAD_RSCALE), (f16) (v1 * EXL3_HAD_RSCALE) };
    *to_global_w((uint32_t*) (dst + col)) = as_u32(o);
}

// ---- run table (exl3_moe_coop_kernel.cuh:273-356): active slots sorted by (local expert, slot),
// runs of at most ROWS slots of one expert.  Layout [n_runs, -, run_start[slots_max + 1],
// order[slots_max]].  One workgroup of NT >= slots threads.
__device__ __forceinline__ void build_runs(const MoeArgs& a)
{
    __shared__ int sh_local[256];
    __shared__ int sh_order[256];
    __shared__ int sh_cnt[NW];
    __shared__ int sh_nact;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int slots = a.bsz * a.topk;
    int* run_start = a.runs + 2;
    int* order = a.runs + 2 + a.slots_max + 1;
    if (t < slots)
    {
        const SlotInfo si = slot_info(a, t);
        sh_local[t] = si.active ? si.local : -1;
    }
    if (t == 0) sh_nact = 0;
    __syncthreads();
    if (t < slots && sh_local[t] >= 0)
    {
        const int e = sh_local[t];
        int rank = 0;
        for (int u = 0; u < slots; ++u)
        {
            const int eu = sh_local[u];
            rank += (eu >= 0 && (eu < e || (eu == e && u < t))) ? 1 : 0;
        }
        sh_order[rank] = t;
        atomicMax(&sh_nact, rank + 1);
    }
    __syncthreads();
    const int n_active = sh_nact;
    int is_start = 0;
    if (t < n_active)
    {
        const int e_t = sh_local[sh_order[t]];
        int first = 0;
        for (int u = 0; u < slots; ++u)
        {
            const int eu = sh_local[u];
            first += (eu >= 0 && eu < e_t) ? 1 : 0;
        }
        is_start = (t == 0 || sh_local[sh_order[t - 1]] != e_t || (t - first) % ROWS == 0) ? 1 : 0;
        *to_global_w(order + t) = sh_order[t];
    }
    const uint64_t bal = __ballot(is_start);
    const int prefix = __popcll(bal & ((1ull << lane) - 1));
    if (lane == 0) sh_cnt[wave] = __popcll(bal);
    __syncthreads();
    int base = 0, total = 0;
    for (int w = 0; w < NW; ++w)
    {
        if (w < wave) base += sh_cnt[w];
        total += sh_cnt[w];
    }
    if (is_start) *to_global_w(run_start + base + prefix) = t;
    if (t == 0)
    {
        *to_global_w(run_start + total) = n_active;
        *to_global_w(a.runs) = total;
    }
}

__global__ __launch_bounds__(NT)
void moe_route_kernel(const MoeArgs a)
{
    if (blockIdx.x == 0) build_runs(a);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nproj = a.gated ? 2 : 1;
    const int chunks = a.Hi / 128;
    const int slots = a.bsz * a.topk;
    const int item = blockIdx.x * NW + wave;
    if (item >= slots * chunks * nproj) return;
    const int s = item / (chunks * nproj);
    const int rem = item % (chunks * nproj);
    const int c = rem / nproj;
    const bool is_gate = a.gated && (rem % nproj) == 0;
    const SlotInfo si = slot_info(a, s);
    if (!si.active)
    {
        if (rem % nproj == 0 && s % a.topk == 0 && token_active_slots(a, si.row) == 0)
            for (int oc = c; oc < a.Ho / 128; oc += chunks) write_empty_row_chunk(a, si.row, oc, lane);
        return;
    }
    const uint16_t* suh = tab<uint16_t>(is_gate ? a.g_suh : a.u_suh, si.local);
    uint16_t* dst = (is_gate ? a.had_g : a.had_u) + (size_t) s * a.Hi;
    rotate_chunk(a, si.row, suh, c, dst, lane);
}

// Where a run's x rows come from: rows[r] of `src`, row stride `ld` (fp16).
struct XSrc
{
    const uint16_t* src;
    int ld;
    const int* rows;
};

// x rows of the run (fp16 rows of `src`, row stride `ld`) for k-slices [ks0, ks0 + nks) into LDS
// as (x, x) pairs (DUP) or as they are (the MUL1 body dots packed weight pairs).  16-byte loads, two per thread in flight before either is consumed: one
// memory round trip per 2 x 256 x 8 halves instead of one per pair.
template <bool DUP>
__device__ __forceinline__ void stage_x(const uint16_t* src, int ld, const int* rows, int nrows, int ks0, int nks,
                                        uint32_t* xs, int xs_stride)
{
    constexpr int B = 2;
    const int per_row = nks * 2;                          // 16-byte groups (8 halves) per row
    const int total = nrows * per_row;
    for (int e0 = 0; e0 < total; e0 += NT * B)
    {
        u32x4 v[B];
        #pragma unroll
        for (int j = 0; j < B; ++j)
        {
            const int e = min(e0 + j * NT + (int) threadIdx.x, total - 1);
            const int r = e / per_row, i = e - r * per_row;
            v[j] = *to_global((const u32x4*) (src + (size_t) rows[r] * ld + ks0 * 16) + i);
        }
        #pragma unroll
        for (int j = 0; j < B; ++j)
        {
            const int e = e0 + j * NT + (int) threadIdx.x;
            const int r = e / per_row, i = e - r * per_row;
            if (e < total && !DUP) *(u32x4*) (xs + r * xs_stride + 4 * i) = v[j];
            if (e < total && DUP)
            {
                uint32_t* d = xs + r * xs_stride + 8 * i;
                const uint32_t w[4] = { v[j].x, v[j].y, v[j].z, v[j].w };
                uint32_t o[8];
                #pragma unroll
                for (int t = 0; t < 4; ++t)
                {
                    const f16x2 h = as_h2(w[t]);
                    const f16x2 d0 = { h.x, h.x }, d1 = { h.y, h.y };
                    o[2 * t] = as_u32(d0);
                    o[2 * t + 1] = as_u32(d1);
                }
                *(u32x4*) d = (u32x4) { o[0], o[1], o[2], o[3] };
                *(u32x4*) (d + 4) = (u32x4) { o[4], o[5], o[6], o[7] };
            }
        }
    }
    __syncthreads();
}

// ---- the multi-row GEMV of one workgroup: rows = the run's slots (x in LDS as (x, x) pairs,
// xs[r * xs_stride + i] for k-slices [ks0, ks0 + nks)), one 128-column chunk of the expert's
// trellis.  Same decode and v_dot2 as the dense GEMV.  Leaves res[r][128] fp32 (MUL1 affine
// correction applied).
template <int K, int CB, int MT>
__device__ __forceinline__ void moe_gemv(const uint16_t* trellis, int tiles_n, int chunk, int ks0, int nks,
                         const XSrc& xsrc, uint32_t* xs, int xs_stride, int nrows, float* red, float* res)
{
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t a3 = sconst(89226354u), b3 = vconst(64248484u);
    const int myn = nks > wave ? (nks - wave + NW - 1) / NW : 0;
    constexpr int KB = kbits(K);                          // whole words per lane (rate code K)
    const size_t kstride = (size_t) NW * tiles_n * tile_words(K);
    const uint32_t* base = (const uint32_t*) trellis + lane_word_off<K>(lane)
                         + ((size_t) (ks0 + min(wave, nks - 1)) * tiles_n + chunk * 8) * tile_words(K);
    constexpr int PF = (MT == 1 && KB <= 4) ? EXL3_MOE_PF1 : 2;
    const int last_i = myn > 0 ? myn - 1 : 0;
    const int prev_off = (lane & 7) == 0 ? 8 * K - 1 : -1;
    uint32_t ring[PF][KB + 1];
    // issued in ring order (the scheduler may not interleave them): the loop head's wait for
    // ring[0] then leaves PF - 1 slices in flight on every path into it
    #pragma unroll
    for (int d = 0; d < PF; ++d)
    {
        load_slot_k<K>(base + (size_t) min(d, last_i) * kstride, prev_off, lane, ring[d]);
        __builtin_amdgcn_sched_barrier(0);
    }
    // the x rows after the weight prefetch: both latencies overlap
    stage_x<CB != 2>(xsrc.src, xsrc.ld, xsrc.rows, min(nrows, MT), ks0, nks, xs, xs_stride);   // LDS holds MT rows

    float acc[MT][2];
    #pragma unroll
    for (int r = 0; r < MT; ++r) acc[r][0] = acc[r][1] = 0.0f;

    for (int i0 = 0; i0 < myn; i0 += PF)
    {
        #pragma unroll
        for (int d = 0; d < PF; ++d)
        {
            const int i = i0 + d;
            const bool live = i < myn;
            const int xo = (wave + min(i, last_i) * NW) * 16;
            uint32_t wv[KB + 1];
            #pragma unroll
            for (int w = 0; w <= KB; ++w) wv[w] = ring[d][w];
            if constexpr (CB == 2)
            {
                // MUL1: the weights of rows 2g and 2g + 1 of a column packed in one word by
                // v_sad_u8 / v_sad_hi_u8 (each half 0x6400 + byte sum, codebook.cuh:78-84),
                // dotted with the x pair (x_2g, x_2g+1): one v_dot2 per two weights
                uint32_t pk[16];
                mul1_pairs<K>(wv, pk);
                load_slot_k<K>(base + (size_t) min(i + PF, last_i) * kstride, prev_off, lane, ring[d]);
                #pragma unroll
                for (int r = 0; r < MT; ++r)
                {
                    if (MT > 1 && r >= nrows) break;
                    const u32x4* xp = (const u32x4*) (xs + r * xs_stride + xo / 2);
                    uint32_t x8[8];
                    #pragma unroll
                    for (int q = 0; q < 2; ++q)
                    {
                        u32x4 tq = xp[q];
                        x8[4 * q] = live ? tq.x : 0u;     x8[4 * q + 1] = live ? tq.y : 0u;
                        x8[4 * q + 2] = live ? tq.z : 0u; x8[4 * q + 3] = live ? tq.w : 0u;
                    }
                    #pragma unroll
                    for (int q = 0; q < 16; ++q)
                    {
                        const int w = 2 * q, gq = w >> 3, jj = w & 7;
                        const int pr = gq + 4 * ((jj >> 1) & 1);        // x pair of rows 2 pr, 2 pr + 1
                        float& acc_ = acc[r][jj >> 2];
                        acc_ = __builtin_amdgcn_fdot2(as_h2(x8[pr]), as_h2(pk[q]), acc_, false);
                    }
                }
            }
            else
            {
            uint32_t raw[32];
            raw32<K, CB>(wv, raw, a3, b3);
            load_slot_k<K>(base + (size_t) min(i + PF, last_i) * kstride, prev_off, lane, ring[d]);
            #pragma unroll
            for (int r = 0; r < MT; ++r)
            {
                if (MT > 1 && r >= nrows) break;
                const u32x4* xp = (const u32x4*) (xs + r * xs_stride + xo);
                uint32_t x16[16];
                #pragma unroll
                for (int q = 0; q < 4; ++q)
                {
                    u32x4 tq = xp[q];
                    x16[4 * q] = live ? tq.x : 0u;     x16[4 * q + 1] = live ? tq.y : 0u;
                    x16[4 * q + 2] = live ? tq.z : 0u; x16[4 * q + 3] = live ? tq.w : 0u;
                }
                #pragma unroll
                for (int w = 0; w < 32; ++w)
                {
                    const int gq = w >> 3, jj = w & 7;
                    const int row = 2 * gq + (jj & 1) + 8 * ((jj >> 1) & 1);
                    float& acc_ = acc[r][jj >> 2];
                    acc_ = __builtin_amdgcn_fdot2(as_h2(x16[row]), as_h2(raw[w]), acc_, false);
                }
            }
            }
        }
    }
    const int c0 = (lane >> 3) * 16 + (lane & 7);
    #pragma unroll
    for (int r = 0; r < MT; ++r)
    {
        if (MT > 1 && r >= nrows) break;
        red[(wave * MT + r) * 128 + c0] = acc[r][0];
        red[(wave * MT + r) * 128 + c0 + 8] = acc[r][1];
    }
    __shared__ float sumx[ROWS];
    if (CB == 2)
    {
        for (int r = wave; r < nrows; r += NW)
        {
            float sv = 0.0f;
            for (int e = lane; e < nks * 8; e += 64)
            {
                const f16x2 h = as_h2(xs[r * xs_stride + e]);
                sv += (float) h.x + (float) h.y;
            }
            sv = wave_sum(sv, lane);
            if (lane == 0) sumx[r] = sv;
        }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < nrows * 128; e += NT)
    {
        const int r = e >> 7, c = e & 127;
        float v = 0.0f;
        #pragma unroll
        for (int w = 0; w < NW; ++w) v += red[(w * MT + r) * 128 + c];
        if (CB == 2) v = v * (float) as_h(0x1eee) + sumx[r] * (float) as_h(0xc931);
        res[r * 128 + c] = v;
    }
    __syncthreads();
}

// HS: the half-rate variant (rate codes 16 + b, mul1 only), a launch of its own so that the
// integer-rate kernels keep their register budget.
template <int CB, int MT, bool HS>
__device__ __forceinline__ void moe_gemv_k(int bits, const uint16_t* trellis, int tiles_n, int chunk, int ks0, int nks,
                           const XSrc& xsrc, uint32_t* xs, int xs_stride, int nrows, float* red, float* res)
{
    if constexpr (HS)
    {
        if (bits == 17) moe_gemv<17, CB, MT>(trellis, tiles_n, chunk, ks0, nks, xsrc, xs, xs_stride, nrows, red, res);
        else if (bits == 18) moe_gemv<18, CB, MT>(trellis, tiles_n, chunk, ks0, nks, xsrc, xs, xs_stride, nrows, red, res);
        else moe_gemv<19, CB, MT>(trellis, tiles_n, chunk, ks0, nks, xsrc, xs, xs_stride, nrows, red, res);
        return;
    }
    else
    {
        switch (bits)
        {
            case 1: moe_gemv<1, CB, MT>(trellis, tiles_n, chunk, ks0, nks, xsrc, xs, xs_stride, nrows, red, res); break;
            case 2: moe_gemv<2, CB, MT>(trellis, tiles_n, chunk, ks0, nks, xsrc, xs, xs_stride, nrows, red, res); break;
            case 3: moe_gemv<3, CB, MT>(trellis, tiles_n, chunk, ks0, nks, xsrc, xs, xs_stride, nrows, red, res); break;
            case 4: moe_gemv<4, CB, MT>(trellis, tiles_n, chunk, ks0, nks, xsrc, xs, xs_stride, nrows, red, res); break;
            case 5: moe_gemv<5, CB, MT>(trellis, tiles_n, chunk, ks0, nks, xsrc, xs, xs_stride, nrows, red, res); break;
            case 6: moe_gemv<6, CB, MT>(trellis, tiles_n, chunk, ks0, nks, xsrc, xs, xs_stride, nrows, red, res); break;
            case 7: moe_gemv<7, CB, MT>(trellis, tiles_n, chunk, ks0, nks, xsrc, xs, xs_stride, nrows, red, res); break;
            default: moe_gemv<8, CB, MT>(trellis, tiles_n, chunk, ks0, nks, xsrc, xs, xs_stride, nrows, red, res); break;
        }
    }
}

// Hand-off of every row of a run at once: each thread waits for its partial stores, the
// workgroup releases them, then thread r < nrows counts row r in counter ctr_r (total arrivals
// total_r), re-arming it when its arrival is the last; last[r] tells the epilogue which rows this
// workgroup completes.  One counter round trip for the run instead of one per row.
template <typename CtrOf>
__device__ __forceinline__ void arrive_rows(int nrows, CtrOf ctr_of, int* last, bool xcd, const XcdGuard& q)
{
    if (xcd) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (xcd) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    else __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if ((int) threadIdx.x < nrows)
    {
        int total;
        int* ctr = ctr_of((int) threadIdx.x, total);
        bool done;
        if (xcd) done = xcd_arrive(q, ctr, total);      // 64-bit counter with the XCC record
        else
        {
            done = __hip_atomic_fetch_add(to_global_w(ctr), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == total - 1;
            if (done) __hip_atomic_store(to_global_w(ctr), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        last[threadIdx.x] = done;
    }
    __syncthreads();
}

__device__ __forceinline__ void acquire_handoff(bool xcd)
{
    if (xcd) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    else __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

// device-scope load (misses L1): data another workgroup of this launch wrote
__device__ __forceinline__ f32x2 load_l2_f32x2(const float* p)
{
    return __builtin_bit_cast(f32x2, __hip_atomic_load(to_global((const uint64_t*) p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// workgroup -> (chunk, rest): chunk c on XCD c % xcd when enabled
__device__ __forceinline__ void chunk_coords(int xcd, int chunks, int& chunk, int& rest)
{
    moe_chunk_coords(xcd, chunks, (int) blockIdx.x, chunk, rest);
}

__device__ __forceinline__ bool read_run(const MoeArgs& a, int run, int* rows, int& nrows)
{
    const int n_runs = *to_global(a.runs);
    if (run >= n_runs) return false;
    const int start = *to_global(a.runs + 2 + run), end = *to_global(a.runs + 3 + run);
    nrows = end - start;
    if ((int) threadIdx.x < nrows) rows[threadIdx.x] = *to_global(a.runs + 2 + a.slots_max + 1 + start + threadIdx.x);
    __syncthreads();
    return true;
}

constexpr int UP_PF_SPLITS = 4;          // k-splits whose partials the gate/up epilogue prefetches

template <int CB, int MT, bool HS>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(CB == 2 ? (MT == 1 ? 4 : 3) : 1)))
void moe_a_kernel(const MoeArgs a)
{
    extern __shared__ __align__(16) uint32_t smem[];
    __shared__ int rows[ROWS];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nproj = a.gated ? 2 : 1;
    const int chunks = a.I / 128;
    const int slots = a.bsz * a.topk;
    const int S = a.splits_a;
    int chunk, rest;
    chunk_coords(a.xcd, chunks, chunk, rest);
    const int q = rest % S;
    const int pr = (rest / S) % nproj;
    const int run = rest / S / nproj;
    const bool is_gate = a.gated && pr == 0;
    int nrows = 0;
    if (!read_run(a, run, rows, nrows)) return;
    if (nrows <= a.run_lo || nrows > a.run_hi) return;  // another launch's size class
    const int local = slot_info(a, rows[0]).local;
    const int bits = a.g_bits ? (int) *to_global((is_gate ? a.g_bits : a.u_bits) + local) : a.K_gu;
    const int KS = a.Hi / 16;
    const int ks0 = KS * q / S, nks = KS * (q + 1) / S - ks0;
    const int xs_stride = SBMAX * 16 + 4;
    uint32_t* xs = smem;
    float* red = (float*) (smem + MT * xs_stride);     // LDS sized for MT rows (moe_lds_bytes)
    float* res = red + NW * MT * 128;
    // MT rows per pass (a run larger than MT, possible only in the single-row launch of a
    // one-token batch with a repeated expert, takes several passes over the weights)
    for (int r0 = 0; r0 < (MT == 1 ? nrows : 1); r0 += MT)
    {
        const int nr = min(MT, nrows - r0);
        const XSrc xsrc = { is_gate ? a.had_g : a.had_u, a.Hi, rows + r0 };
        moe_gemv_k<CB, MT, HS>(bits, tab<uint16_t>(is_gate ? a.g_trellis : a.u_trellis, local), a.I / 16, chunk, ks0,
                           nks, xsrc, xs, xs_stride, nr, red, res);
        // split partials: part_a[proj][split][slot][I]
        for (int e = threadIdx.x; e < nr * 64; e += NT)
        {
            const int r = e >> 6, c2 = e & 63;
            float* dst = a.part_a + (((size_t) pr * S + q) * slots + rows[r0 + r]) * a.I + chunk * 128 + 2 * c2;
            *to_global_w((f32x2*) dst) = *(const f32x2*) (res + r * 128 + 2 * c2);
        }
    }
    // completed (slot, chunk) rows: one wave each
    __shared__ int last[ROWS];
    arrive_rows(nrows, [&](int r, int& total) { total = nproj * S; return a.ctr_a + ((size_t) rows[r] * chunks + chunk) * 32; },
                last, a.xcd > 0, a.xg);
    for (int r = wave; r < nrows; r += NW)
    {
        if (!last[r]) continue;
        acquire_handoff(a.xcd > 0);
        const int s = rows[r];
        {
            const int col = chunk * 128 + 2 * lane;
            // every load of the epilogue issued before the first is consumed (split partials of
            // up and gate, svh / bias / down-suh pairs): one round trip instead of a chain.  The
            // sums run in the order of the general loop (slot order from 0.0f), so the bits are
            // the same; more than UP_PF_SPLITS splits take the general loop.
            const int pu_idx = a.gated ? 1 : 0;
            f32x2 pu[UP_PF_SPLITS], pg[UP_PF_SPLITS];
            const bool pf = S <= UP_PF_SPLITS && !a.epi_serial;
            if (pf)
            {
                #pragma unroll
                for (int qq = 0; qq < UP_PF_SPLITS; ++qq)
                {
                    const int qc = min(qq, S - 1);
                    pu[qq] = load_l2_f32x2(a.part_a + (((size_t) pu_idx * S + qc) * slots + s) * a.I + col);
                    // (ungated: the up partials again, unused)
                    pg[qq] = load_l2_f32x2(a.part_a + (((size_t) 0 * S + qc) * slots + s) * a.I + col);
                }
            }
            const uint16_t* usvh = tab<uint16_t>(a.u_svh, local);
            const uint16_t* dsuh = tab<uint16_t>(a.d_suh, local);
            const float us0 = h2f(usvh, col), us1 = h2f(usvh, col + 1);
            const float ds0 = h2f(dsuh, col), ds1 = h2f(dsuh, col + 1);
            float gs0 = 0.0f, gs1 = 0.0f;
            if (a.gated)            // the gate tables are read only for a gated MoE
            {
                const uint16_t* gsvh = tab<uint16_t>(a.g_svh, local);
                gs0 = h2f(gsvh, col); gs1 = h2f(gsvh, col + 1);
            }
            float ub0 = 0.0f, ub1 = 0.0f, gb0 = 0.0f, gb1 = 0.0f;
            if (a.u_bias) { const uint16_t* b = tab<uint16_t>(a.u_bias, local); ub0 = h2f(b, col); ub1 = h2f(b, col + 1); }
            if (a.gated && a.g_bias) { const uint16_t* b = tab<uint16_t>(a.g_bias, local); gb0 = h2f(b, col); gb1 = h2f(b, col + 1); }
            auto load_sum = [&](int p, const f32x2* pv, float& v0, float& v1) {
                v0 = v1 = 0.0f;
                if (pf)
                {
                    #pragma unroll
                    for (int qq = 0; qq < UP_PF_SPLITS; ++qq)
                        if (qq < S) { v0 += pv[qq].x; v1 += pv[qq].y; }
                    return;
                }
                for (int qq = 0; qq < S; ++qq)
                {
                    const f32x2 t = load_l2_f32x2(a.part_a + (((size_t) p * S + qq) * slots + s) * a.I + col);
                    v0 += t.x; v1 += t.y;
                }
            };
            float u0, u1;
            load_sum(pu_idx, pu, u0, u1);
            fwht128_wave(u0, u1, lane);
            u0 *= EXL3_HAD_RSCALE; u1 *= EXL3_HAD_RSCALE;
            u0 *= us0; u1 *= us1;
            if (a.u_bias) { u0 += ub0; u1 += ub1; }
            float g0 = u0, g1 = u1;
            if (a.gated)
            {
                load_sum(0, pg, g0, g1);
                fwht128_wave(g0, g1, lane);
                g0 *= EXL3_HAD_RSCALE; g1 *= EXL3_HAD_RSCALE;
                g0 *= gs0; g1 *= gs1;
                if (a.g_bias) { g0 += gb0; g1 += gb1; }
            }
            float a0 = act_gate(a.act, a.gated, g0, u0, a.act_limit);
            float a1 = act_gate(a.act, a.gated, g1, u1, a.act_limit);
            a0 *= ds0; a1 *= ds1;
            fwht128_wave(a0, a1, lane);
            const f16x2 o = { (f16) (a0 * EXL3_HAD_RSCALE), (f16) (a1 * EXL3_HAD_RSCALE) };
            *to_global_w((uint32_t*) (a.act_out + (size_t) s * a.I + col)) = as_u32(o);
        }
    }
}

// The down epilogue's slot sum for top-k <= WKR (every partition holds at most slot k = w) and
// at most DOWN_PF_SPLITS k-splits: the same arithmetic, in the same order, as the general loop in
// moe_b_kernel, but each group of DOWN_PF_SLOTS slots issues all its loads (routing, split
// partials, svh and bias pairs) before the first is consumed, so that the group costs one chain
// of dependent round trips instead of one per slot.  Loads are clamped and unconditional.
constexpr int DOWN_PF_SLOTS = 8, DOWN_PF_SPLITS = 2;

__device__ __forceinline__ void down_sum_prefetched(const MoeArgs& a, int row, int col, int lane, int S,
                                                    float& o0, float& o1)
{
    const int slots = a.bsz * a.topk;
    for (int k0 = 0; k0 < WKR; k0 += DOWN_PF_SLOTS)
    {
        if (k0 >= a.topk)
        {
            // partitions without a slot add p = 0 (o + 0 is idempotent after the first)
            o0 += 0.0f;
            o1 += 0.0f;
            continue;
        }
        SlotInfo sj[DOWN_PF_SLOTS];
        f32x2 pt[DOWN_PF_SLOTS][DOWN_PF_SPLITS];
        float sv0[DOWN_PF_SLOTS], sv1[DOWN_PF_SLOTS], bv0[DOWN_PF_SLOTS], bv1[DOWN_PF_SLOTS];
        #pragma unroll
        for (int u = 0; u < DOWN_PF_SLOTS; ++u)
            sj[u] = slot_info(a, row * a.topk + min(k0 + u, a.topk - 1));
        #pragma unroll
        for (int u = 0; u < DOWN_PF_SLOTS; ++u)
        {
            const int sk = row * a.topk + min(k0 + u, a.topk - 1);
            #pragma unroll
            for (int qq = 0; qq < DOWN_PF_SPLITS; ++qq)
                pt[u][qq] = load_l2_f32x2(a.part_b + ((size_t) min(qq, S - 1) * slots + sk) * a.Ho + col);
        }
        #pragma unroll
        for (int u = 0; u < DOWN_PF_SLOTS; ++u)
        {
            const uint16_t* dsvh = tab<uint16_t>(a.d_svh, sj[u].local);
            sv0[u] = h2f(dsvh, col); sv1[u] = h2f(dsvh, col + 1);
            bv0[u] = 0.0f; bv1[u] = 0.0f;
            if (a.d_bias)
            {
                const uint16_t* bp = tab<uint16_t>(a.d_bias, sj[u].local);
                bv0[u] = h2f(bp, col); bv1[u] = h2f(bp, col + 1);
            }
        }
        #pragma unroll
        for (int u = 0; u < DOWN_PF_SLOTS; ++u)
        {
            const int k = k0 + u;                      // partition w = k
            float p0 = 0.0f, p1 = 0.0f;
            if (k < a.topk && sj[u].active)
            {
                float v0 = 0.0f, v1 = 0.0f;
                #pragma unroll
                for (int qq = 0; qq < DOWN_PF_SPLITS; ++qq)
                    if (qq < S) { v0 += pt[u][qq].x; v1 += pt[u][qq].y; }
                fwht128_wave(v0, v1, lane);
                v0 *= EXL3_HAD_RSCALE; v1 *= EXL3_HAD_RSCALE;
                v0 *= sv0[u]; v1 *= sv1[u];
                if (a.d_bias) { v0 += bv0[u]; v1 += bv1[u]; }
                p0 += sj[u].w * v0;
                p1 += sj[u].w * v1;
            }
            o0 += p0;
            o1 += p1;
        }
    }
}

template <int CB, int MT, bool HS>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(CB == 2 ? (MT == 1 ? 4 : 3) : 1)))
void moe_b_kernel(const MoeArgs a)
{
    extern __shared__ __align__(16) uint32_t smem[];
    __shared__ int rows[ROWS];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int chunks = a.Ho / 128;
    const int slots = a.bsz * a.topk;
    const int S = a.splits_b;
    int chunk, rest;
    chunk_coords(a.xcd, chunks, chunk, rest);
    const int q = rest % S;
    const int run = rest / S;
    int nrows = 0;
    if (!read_run(a, run, rows, nrows)) return;
    if (nrows <= a.run_lo || nrows > a.run_hi) return;  // another launch's size class
    const int local = slot_info(a, rows[0]).local;
    const int bits = a.d_bits ? (int) *to_global(a.d_bits + local) : a.K_d;
    const int KS = a.I / 16;
    const int ks0 = KS * q / S, nks = KS * (q + 1) / S - ks0;
    const int xs_stride = SBMAX * 16 + 4;
    uint32_t* xs = smem;
    float* red = (float*) (smem + MT * xs_stride);     // LDS sized for MT rows (moe_lds_bytes)
    float* res = red + NW * MT * 128;
    for (int r0 = 0; r0 < (MT == 1 ? nrows : 1); r0 += MT)
    {
        const int nr = min(MT, nrows - r0);
        const XSrc xsrc = { a.act_out, a.I, rows + r0 };
        moe_gemv_k<CB, MT, HS>(bits, tab<uint16_t>(a.d_trellis, local), a.Ho / 16, chunk, ks0, nks, xsrc, xs, xs_stride,
                           nr, red, res);
        for (int e = threadIdx.x; e < nr * 64; e += NT)
        {
            const int r = e >> 6, c2 = e & 63;
            float* dst = a.part_b + ((size_t) q * slots + rows[r0 + r]) * a.Ho + chunk * 128 + 2 * c2;
            *to_global_w((f32x2*) dst) = *(const f32x2*) (res + r * 128 + 2 * c2);
        }
    }
    // completed (token, chunk) outputs: one wave each (a token with two slots in this run
    // arrives twice; only one arrival can be the last)
    __shared__ int last[ROWS];
    arrive_rows(nrows, [&](int r, int& total) {
                    const int row = rows[r] / a.topk;
                    total = token_active_slots(a, row) * S;
                    return a.ctr_b + ((size_t) row * chunks + chunk) * 32; },
                last, a.xcd > 0, a.xg);
    for (int r = wave; r < nrows; r += NW)
    {
        if (!last[r]) continue;
        acquire_handoff(a.xcd > 0);
        const int row = rows[r] / a.topk;
        {
            const int col = chunk * 128 + 2 * lane;
            float o0 = 0.0f, o1 = 0.0f;
            // slots k = w, w + 16, ... summed per w, then the partitions in order (:960-979)
            if (a.topk <= WKR && S <= DOWN_PF_SPLITS && !a.epi_serial)
                down_sum_prefetched(a, row, col, lane, S, o0, o1);
            else
            for (int w = 0; w < WKR; ++w)
            {
                float p0 = 0.0f, p1 = 0.0f;
                for (int k = w; k < a.topk; k += WKR)
                {
                    const int sk = row * a.topk + k;
                    const SlotInfo sj = slot_info(a, sk);
                    if (!sj.active) continue;
                    float v0 = 0.0f, v1 = 0.0f;
                    for (int qq = 0; qq < S; ++qq)
                    {
                        const f32x2 t = load_l2_f32x2(a.part_b + ((size_t) qq * slots + sk) * a.Ho + col);
                        v0 += t.x; v1 += t.y;
                    }
                    fwht128_wave(v0, v1, lane);
                    v0 *= EXL3_HAD_RSCALE; v1 *= EXL3_HAD_RSCALE;
                    const uint16_t* dsvh = tab<uint16_t>(a.d_svh, sj.local);
                    v0 *= h2f(dsvh, col); v1 *= h2f(dsvh, col + 1);
                    if (a.d_bias)
                    {
                        const uint16_t* b = tab<uint16_t>(a.d_bias, sj.local);
                        v0 += h2f(b, col); v1 += h2f(b, col + 1);
                    }
                    p0 += sj.w * v0;
                    p1 += sj.w * v1;
                }
                o0 += p0;
                o1 += p1;
            }
            if (a.sh_out)
            {
                const float gv = a.sh_gate_w ? shared_gate(a, row, lane) : 1.0f;
                const float* sh = a.sh_out + (size_t) row * a.H + col;
                if (col < a.H) o0 += gv * *to_global(sh);
                if (col + 1 < a.H) o1 += gv * *to_global(sh + 1);
            }
            float* dst = a.out + (size_t) row * a.out_stride + col;
            if (col < a.H_out) *to_global_w(dst) = o0;
            if (col + 1 < a.H_out) *to_global_w(dst + 1) = o1;
        }
    }
}

}  // namespace

// Launch the three stages.  Dynamic LDS: x pairs + the wave reduction + the result rows.
#define EXL3_CAT2(a, b) a##b
#define EXL3_CAT(a, b) EXL3_CAT2(a, b)

int EXL3_CAT(exl3k_moe_cb, EXL3_MOE_CB)(const MoeArgs& a, hipStream_t s)
{
    const int nproj = a.gated ? 2 : 1;
    const int slots = a.bsz * a.topk;
    // x rows + the wave reduction + the result rows, for MT rows: the single-row variant needs
    // 6.7 KB instead of 53 KB, so LDS no longer caps it at 3 workgroups per CU
    auto moe_lds_bytes = [](int mt) { return ((size_t) mt * (SBMAX * 16 + 4) + (size_t) NW * mt * 128 + (size_t) mt * 128) * 4; };
    const int rot_items = slots * (a.Hi / 128) * nproj;
    hipLaunchKernelGGL(moe_route_kernel, dim3((rot_items + NW - 1) / NW), dim3(NT), 0, s, a);
    // Runs by size class, each with the GEMV body of its row count: VGPRs (126 for one row, 204
    // for eight) set the waves per SIMD, and most runs of a decode batch hold a single slot.  A
    // one-token batch has distinct picks but for repeats, so its single-row launch takes every
    // run (a repeat costs a second pass) and the eight-row launch is skipped.
    const int gridA = slots * (a.I / 128) * nproj * a.splits_a, gridB = slots * (a.Ho / 128) * a.splits_b;
    const bool multi = a.bsz > 1;
    MoeArgs c1 = a, c8 = a;
    c1.run_lo = 0; c1.run_hi = multi ? 1 : ROWS;
    c8.run_lo = 1; c8.run_hi = ROWS;
#if EXL3_MOE_CB == 2
    if (a.K_gu >= 16 && !a.g_bits)
    {
        hipLaunchKernelGGL((moe_a_kernel<EXL3_MOE_CB, 1, true>), dim3(gridA), dim3(NT), moe_lds_bytes(1), s, c1);
        if (multi) hipLaunchKernelGGL((moe_a_kernel<EXL3_MOE_CB, ROWS, true>), dim3(gridA), dim3(NT), moe_lds_bytes(ROWS), s, c8);
    }
    else
#endif
    {
        hipLaunchKernelGGL((moe_a_kernel<EXL3_MOE_CB, 1, false>), dim3(gridA), dim3(NT), moe_lds_bytes(1), s, c1);
        if (multi) hipLaunchKernelGGL((moe_a_kernel<EXL3_MOE_CB, ROWS, false>), dim3(gridA), dim3(NT), moe_lds_bytes(ROWS), s, c8);
    }
#if EXL3_MOE_CB == 2
    if (a.K_d >= 16 && !a.d_bits)
    {
        hipLaunchKernelGGL((moe_b_kernel<EXL3_MOE_CB, 1, true>), dim3(gridB), dim3(NT), moe_lds_bytes(1), s, c1);
        if (multi) hipLaunchKernelGGL((moe_b_kernel<EXL3_MOE_CB, ROWS, true>), dim3(gridB), dim3(NT), moe_lds_bytes(ROWS), s, c8);
    }
    else
#endif
    {
        hipLaunchKernelGGL((moe_b_kernel<EXL3_MOE_CB, 1, false>), dim3(gridB), dim3(NT), moe_lds_bytes(1), s, c1);
        if (multi) hipLaunchKernelGGL((moe_b_kernel<EXL3_MOE_CB, ROWS, false>), dim3(gridB), dim3(NT), moe_lds_bytes(ROWS), s, c8);
    }
    return (int) hipGetLastError();
}
