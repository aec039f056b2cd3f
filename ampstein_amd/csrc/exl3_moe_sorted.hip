// Token-sorted MoE for prefill-sized batches (exl3_moe, quant/exl3_moe.cu:137-418, kernel
// exl3_moe_kernel.cuh:78-313) and its fixed-order reduction (exl3_moe_gather, exl3_moe.cu:420-531).
//
// The reference runs one cooperative kernel whose workgroup groups walk the experts with group
// barriers.  Here kernel boundaries are the barriers, and all experts of a call run at once:
//   plan     one workgroup: per-expert starts in the sorted assignment list, the experts this
//            launch takes (0 < count <= max_tokens_per_expert, count_lo <= count <= count_hi),
//            their rows compacted into a pool (the caller's temp buffers, concurrency x
//            max_tokens_per_expert rows), row tiles of <= 64 / 128 / 256 rows of one expert, and per
//            (matrix, bitrate) lists of row tiles;
//   gather   pool row r <- had(x[token] o suh) for gate and up (had_hf_r_128_inner);
//   GEMM     grouped MFMA GEMM (exl3_gemm.hip, GROUP instance) per bitrate, gate and up together;
//   act      had(g) o svh_g, had(u) o svh_u, act, limit, g * u, o suh_d, had (had_hf_r_128_guad_inner);
//   GEMM     down;
//   out      had(d) * (w / sqrt(128)) o svh_d added atomically to the token's row, or stored in its
//            slot of output_scratch (had_hf_r_128_d_inner).
// Rows of one pass are independent, so a pool smaller than the routed rows is run in passes.
// Every 128-chunk is rotated by 16 lanes, 8 elements each, with the reference's butterfly order
// (in-lane widths 1, 2, 4, DPP 8 .. 64), one fp32 rounding per stage: the rotations are
// bit-identical to the reference's shuffle placement.
#include <algorithm>
#include <cstring>

#include "exl3_common.cuh"
#include "exl3_kernels.h"

using namespace exl3;

namespace {

constexpr float R128 = 0.088388347648f;   // 1 / sqrt(128), as the reference spells it
constexpr int PLAN_THREADS = 1024;
constexpr int PLAN_EMAX = 4096;

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

// SW: the partner through the LDS crossbar (ds_swizzle) instead of DPP: one LDS-pipe op instead
// of one or two VALU ops, for the VALU-bound gather and activation kernels (activation 92 -> 80
// us at T = 2048); the output kernel is latency-bound and keeps DPP.
template <int M, bool SW>
__device__ __forceinline__ void fwht8_stage(float* e, int lane)
{
    const float sg = (lane & M) ? -1.0f : 1.0f;
    #pragma unroll
    for (int i = 0; i < 8; ++i)
    {
        const float p = SW ? xor_partner_sw<M>(e[i]) : xor_partner<M>(e[i], lane);
        e[i] = __builtin_fmaf(sg, e[i], p);
    }
}

// H128 of the 16-lane group's chunk (lane g holds elements 8g .. 8g+7), unscaled.
template <bool SW = false>
__device__ __forceinline__ void fwht128_g16(float* e, int lane)
{
    fwht8_inlane(e);
    fwht8_stage<1, SW>(e, lane);
    fwht8_stage<2, SW>(e, lane);
    fwht8_stage<4, SW>(e, lane);
    fwht8_stage<8, SW>(e, lane);
}

__device__ __forceinline__ void unpack8(const u32x4& v, uint32_t* w)
{
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
}

__device__ __forceinline__ void to_f32(const uint32_t* w, float* e)
{
    #pragma unroll
    for (int q = 0; q < 4; ++q)
    {
        const f16x2 h = as_h2(w[q]);
        e[2 * q] = (float) h.x;
        e[2 * q + 1] = (float) h.y;
    }
}

__device__ __forceinline__ void to_h(const float* e, uint32_t* w)
{
    #pragma unroll
    for (int q = 0; q < 4; ++q) w[q] = as_u32((f16x2) { (f16) e[2 * q], (f16) e[2 * q + 1] });
}

__device__ __forceinline__ void hmul4(uint32_t* w, const uint32_t* s)
{
    #pragma unroll
    for (int q = 0; q < 4; ++q) w[q] = as_u32(as_h2(w[q]) * as_h2(s[q]));
}

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *to_global((const u32x4*) p); }

// Sum of the 16-lane group's 128 fp16 values (lane g holds 8), in a fixed order: the row-chunk
// sums the mul1 GEMM needs for its affine map (exl3_gemm.hip moeg_kernel).
__device__ __forceinline__ float group_sum16(const uint32_t* w)
{
    float v = 0.0f;
    #pragma unroll
    for (int q = 0; q < 4; ++q)
    {
        const f16x2 h = as_h2(w[q]);
        v += (float) h.x + (float) h.y;
    }
    #pragma unroll
    for (int m = 1; m < 16; m <<= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// ------------------------------------------------------------------------------- plan
// In-place exclusive scan of n <= PLAN_EMAX ints in LDS by PLAN_THREADS threads (4 per thread).
__device__ int scan_excl(int* a, int n, int* tmp)
{
    const int t = threadIdx.x;
    int loc[4], sum = 0;
    #pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const int j = 4 * t + i;
        loc[i] = j < n ? a[j] : 0;
        sum += loc[i];
    }
    tmp[t] = sum;
    __syncthreads();
    for (int off = 1; off < PLAN_THREADS; off <<= 1)
    {
        const int v = t >= off ? tmp[t - off] : 0;
        __syncthreads();
        tmp[t] += v;
        __syncthreads();
    }
    const int total = tmp[PLAN_THREADS - 1];
    int run = tmp[t] - sum;
    #pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const int j = 4 * t + i;
        if (j < n) a[j] = run;
        run += loc[i];
    }
    __syncthreads();
    return total;
}

__global__ __launch_bounds__(PLAN_THREADS)
void moes_plan_kernel(MoesArgs a, int pass_row0)
{
    __shared__ int s_start[PLAN_EMAX], s_cst[PLAN_EMAX], s_nt[PLAN_EMAX], s_tmp[PLAN_THREADS];
    __shared__ int s_lc[3 * MOES_RATES];
    const int t = threadIdx.x, E = a.num_experts;
    if (t < 3 * MOES_RATES) s_lc[t] = 0;
    for (int e = t; e < E; e += PLAN_THREADS)
    {
        const int64_t c64 = a.expert_count[e];
        const int c = c64 > 0x3fffffff ? 0x3fffffff : (int) (c64 < 0 ? 0 : c64);
        s_start[e] = c;
        const bool ok = c > 0 && c <= a.max_tokens && c >= a.count_lo && c <= a.count_hi;
        s_cst[e] = ok ? c : 0;
    }
    __syncthreads();
    // s_nt holds the eligible counts until the scans are done
    for (int e = t; e < E; e += PLAN_THREADS) s_nt[e] = s_cst[e];
    __syncthreads();
    scan_excl(s_start, E, s_tmp);
    const int total = scan_excl(s_cst, E, s_tmp);
    const int w0 = pass_row0, w1 = pass_row0 + a.pool_rows;
    int lo_r[4], n_r[4];
    #pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const int e = 4 * t + i;
        lo_r[i] = 0; n_r[i] = 0;
        if (e < E)
        {
            const int lo = max(s_cst[e], w0), hi = min(s_cst[e] + s_nt[e], w1);
            lo_r[i] = lo;
            n_r[i] = max(0, hi - lo);
        }
    }
    __syncthreads();
    const int TR = a.tile_rows;
    #pragma unroll
    for (int i = 0; i < 4; ++i) if (4 * t + i < E) s_nt[4 * t + i] = (n_r[i] + TR - 1) / TR;
    __syncthreads();
    scan_excl(s_nt, E, s_tmp);
    // row tiles and the per (matrix, bitrate) lists
    #pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const int e = 4 * t + i;
        if (e >= E || n_r[i] == 0) continue;
        int kb[3];
        kb[0] = a.bits_g ? (int) a.bits_g[e] : a.K_g;
        kb[1] = a.bits_u ? (int) a.bits_u[e] : a.K_u;
        kb[2] = a.bits_d ? (int) a.bits_d[e] : a.K_d;
        for (int j = 0; j * TR < n_r[i]; ++j)
        {
            const int tid = s_nt[e] + j;
            a.rt[3 * tid] = e;
            a.rt[3 * tid + 1] = lo_r[i] - w0 + TR * j;
            a.rt[3 * tid + 2] = min(TR, n_r[i] - TR * j);
            #pragma unroll
            for (int m = 0; m < 3; ++m)
            {
                const int slot = moes_rate_slot(kb[m]);
                if (slot < 0) continue;                    // no instance: the reference's switch runs no case
                const int l = m * MOES_RATES + slot;
                const int pos = atomicAdd(&s_lc[l], 1);
                a.lists[(size_t) l * a.rt_cap + pos] = tid;
            }
        }
    }
    __syncthreads();
    if (t < 3 * MOES_RATES) a.counts[t] = s_lc[t];
    // pool row -> (sorted position, expert, row within the expert); -1 past the pass's rows
    for (int r = t; r < a.pool_rows; r += PLAN_THREADS)
    {
        const int c = w0 + r;
        int info0 = -1, e = 0, j = 0;
        if (c < total)                                     // (rows past the assignment list stay unused)
        {
            int lo = 0, hi = E;                            // last e with s_cst[e] <= c
            while (hi - lo > 1)
            {
                const int mid = (lo + hi) >> 1;
                if (s_cst[mid] <= c) lo = mid; else hi = mid;
            }
            e = lo;
            j = c - s_cst[e];
            info0 = s_start[e] + j;
            if (info0 >= a.num_assign) info0 = -1;
        }
        a.rowinfo[3 * r] = info0;
        if (info0 >= 0 && a.inv_row) a.inv_row[info0] = r;
        a.rowinfo[3 * r + 1] = e;
        a.rowinfo[3 * r + 2] = j;
    }
}

// ------------------------------------------------------------------------------- token lists
// Sorted positions of every token, ascending (one workgroup, once per call), all in LDS:
// count per token (LDS atomics), exclusive scan, scatter through the running offsets, an
// insertion sort of each (top-k long) list -- so that the output kernel sums a token's rows in a
// fixed order -- then coalesced copies out.  LDS: bsz + num_assign + PLAN_THREADS ints (the host
// checks the size).
__global__ __launch_bounds__(PLAN_THREADS)
void moes_tokens_kernel(MoesArgs a)
{
    extern __shared__ __align__(16) int sm[];
    const int t = threadIdx.x, T = a.bsz, N = a.num_assign;
    int* s_cnt = sm;                  // counts, then start offsets, then end offsets
    int* s_pos = sm + T;
    int* s_tmp = sm + T + N;
    for (int i = t; i < T; i += PLAN_THREADS) s_cnt[i] = 0;
    __syncthreads();
    for (int p = t; p < N; p += PLAN_THREADS)
    {
        const int64_t tk = a.token_sorted[p];
        if (tk >= 0 && tk < T) atomicAdd(&s_cnt[tk], 1);
    }
    __syncthreads();
    // blocked exclusive scan: thread t owns tokens [t seg, (t + 1) seg)
    const int seg = (T + PLAN_THREADS - 1) / PLAN_THREADS;
    const int lo = min(T, t * seg), hi = min(T, lo + seg);
    int sum = 0;
    for (int i = lo; i < hi; ++i) sum += s_cnt[i];
    s_tmp[t] = sum;
    __syncthreads();
    for (int off = 1; off < PLAN_THREADS; off <<= 1)
    {
        const int v = t >= off ? s_tmp[t - off] : 0;
        __syncthreads();
        s_tmp[t] += v;
        __syncthreads();
    }
    int run = s_tmp[t] - sum;
    for (int i = lo; i < hi; ++i)
    {
        const int c = s_cnt[i];
        s_cnt[i] = run;
        a.tok_start[i] = run;
        run += c;
    }
    if (t == PLAN_THREADS - 1) a.tok_start[T] = s_tmp[t];
    __syncthreads();
    for (int p = t; p < N; p += PLAN_THREADS)
    {
        const int64_t tk = a.token_sorted[p];
        if (tk >= 0 && tk < T) s_pos[atomicAdd(&s_cnt[tk], 1)] = p;     // s_cnt ends at the list ends
    }
    __syncthreads();
    for (int i = t; i < T; i += PLAN_THREADS)
    {
        const int e1 = s_cnt[i], e0 = i ? s_cnt[i - 1] : 0;
        for (int x = e0 + 1; x < e1; ++x)
        {
            const int v = s_pos[x];
            int y = x - 1;
            while (y >= e0 && s_pos[y] > v) { s_pos[y + 1] = s_pos[y]; --y; }
            s_pos[y + 1] = v;
        }
    }
    __syncthreads();
    const int total = T ? s_cnt[T - 1] : 0;
    for (int i = t; i < total; i += PLAN_THREADS) a.tok_pos[i] = s_pos[i];
}

// ------------------------------------------------------------------------------- gather + rotate
// Row-per-wave elementwise kernels.  Wave w takes pool rows w, w + waves, ...; the row's sorted
// position, expert, token and routing weight are wave-uniform (scalar loads, once per row), and
// the row's 128-column chunks go in batches of 4 EW_B chunks (16 lanes per chunk, 8 values per
// lane) whose loads are all issued before the first butterfly.  The per-chunk arithmetic is the
// chunk-per-job form's, value for value.
constexpr int EW_B = 2;                  // 4-chunk groups per batch

__device__ __forceinline__ int wave_id()
{
    return __builtin_amdgcn_readfirstlane((int) blockIdx.x * 4 + (int) (threadIdx.x >> 6));
}

__global__ __launch_bounds__(256)
void moes_gather_kernel(MoesArgs a)
{
    const int lane = threadIdx.x & 63, g = lane & 15, sub = lane >> 4;
    const int chunks = a.H / 128;
    const int nw = gridDim.x * 4;
    for (int r = wave_id(); r < a.pool_rows; r += nw)
    {
        const int pos = a.rowinfo[3 * r];
        if (pos < 0) continue;                             // (uniform) rows past the pass
        const int e = a.rowinfo[3 * r + 1];
        const int64_t token = a.token_sorted[pos];
        const uint16_t* xrow = a.x + token * a.H;
        const uint16_t* suh_g = a.gated ? (const uint16_t*) a.g_suh[e] : nullptr;
        const uint16_t* suh_u = (const uint16_t*) a.u_suh[e];
        for (int c0 = 0; c0 < chunks; c0 += 4 * EW_B)
        {
            u32x4 xv[EW_B], sv[2][EW_B];
            #pragma unroll
            for (int bq = 0; bq < EW_B; ++bq)
            {
                const int col = 128 * min(c0 + 4 * bq + sub, chunks - 1) + 8 * g;
                xv[bq] = __builtin_nontemporal_load(to_global((const u32x4*) (xrow + col)));
                sv[1][bq] = ld16(suh_u + col);
                if (a.gated) sv[0][bq] = ld16(suh_g + col);
            }
            #pragma unroll
            for (int bq = 0; bq < EW_B; ++bq)
            {
                const int c = c0 + 4 * bq + sub;
                const int col = 128 * min(c, chunks - 1) + 8 * g;
                uint32_t xw[4];
                unpack8(xv[bq], xw);
                #pragma unroll
                for (int m = 0; m < 2; ++m)
                {
                    if (m == 0 && !a.gated) continue;      // non-gated: no gate staging
                    uint32_t w[4], sw[4];
                    unpack8(sv[m][bq], sw);
                    #pragma unroll
                    for (int q = 0; q < 4; ++q) w[q] = xw[q];
                    hmul4(w, sw);                          // fp16 pre-scale
                    float f[8];
                    to_f32(w, f);
                    fwht128_g16<true>(f, lane);
                    #pragma unroll
                    for (int i = 0; i < 8; ++i) f[i] *= R128;
                    to_h(f, w);
                    const float cs = group_sum16(w);
                    if (c < chunks)
                    {
                        *(u32x4*) ((m ? a.ts_u : a.ts_g) + (size_t) r * a.H + col) = (u32x4) { w[0], w[1], w[2], w[3] };
                        if (g == 0) (m ? a.ps_u : a.ps_g)[(size_t) r * chunks + c] = cs;
                    }
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------- activation
__device__ __forceinline__ float silu_f(float x) { return silu_f32(x); }
__device__ __forceinline__ float gelu_f(float x)
{
    return 0.5f * x * (1.0f + tanhf(0.797884560803f * (x + 0.044715f * x * x * x)));
}

__global__ __launch_bounds__(256)
void moes_act_kernel(MoesArgs a)
{
    const int lane = threadIdx.x & 63, g = lane & 15, sub = lane >> 4;
    const int chunks = a.I / 128;
    const int nw = gridDim.x * 4;
    const f16 lim = (f16) a.act_limit;
    for (int r = wave_id(); r < a.pool_rows; r += nw)
    {
        if (a.rowinfo[3 * r] < 0) continue;                // (uniform) rows past the pass
        const int e = a.rowinfo[3 * r + 1];
        const uint16_t* svh_u = (const uint16_t*) a.u_svh[e];
        const uint16_t* svh_g = a.gated ? (const uint16_t*) a.g_svh[e] : nullptr;
        const uint16_t* suh_d = (const uint16_t*) a.d_suh[e];
        for (int c0 = 0; c0 < chunks; c0 += 4 * EW_B)
        {
            u32x4 uv[EW_B], gv[EW_B], su[EW_B], sg[EW_B], sd[EW_B];
            #pragma unroll
            for (int bq = 0; bq < EW_B; ++bq)
            {
                const int col = 128 * min(c0 + 4 * bq + sub, chunks - 1) + 8 * g;
                const size_t idx = (size_t) r * a.I + col;
                uv[bq] = ld16(a.ti_u + idx);
                su[bq] = ld16(svh_u + col);
                sd[bq] = ld16(suh_d + col);
                if (a.gated)
                {
                    gv[bq] = ld16(a.ti_g + idx);
                    sg[bq] = ld16(svh_g + col);
                }
            }
            #pragma unroll
            for (int bq = 0; bq < EW_B; ++bq)
            {
                const int c = c0 + 4 * bq + sub;
                const int col = 128 * min(c, chunks - 1) + 8 * g;
                const size_t idx = (size_t) r * a.I + col;
                // had(u) o svh_u
                uint32_t u[4], gg[4] = { 0u, 0u, 0u, 0u }, s[4];
                float f[8];
                unpack8(uv[bq], u);
                to_f32(u, f);
                fwht128_g16<true>(f, lane);
                #pragma unroll
                for (int i = 0; i < 8; ++i) f[i] *= R128;
                to_h(f, u);
                unpack8(su[bq], s);
                hmul4(u, s);
                if (a.gated)
                {
                    unpack8(gv[bq], gg);
                    to_f32(gg, f);
                    fwht128_g16<true>(f, lane);
                    #pragma unroll
                    for (int i = 0; i < 8; ++i) f[i] *= R128;
                    to_h(f, gg);
                    unpack8(sg[bq], s);
                    hmul4(gg, s);
                }
                // activation of the gate lane, per element in fp32 from the fp16 value, rounded once
                #pragma unroll
                for (int q = 0; q < 4; ++q)
                {
                    f16x2 hg = as_h2(gg[q]);
                    const f16x2 hu = as_h2(u[q]);
                    if (a.act == 0) hg = (f16x2) { (f16) silu_f((float) hg.x), (f16) silu_f((float) hg.y) };
                    else if (a.act == 1) hg = (f16x2) { (f16) gelu_f((float) hg.x), (f16) gelu_f((float) hg.y) };
                    else if (a.act == 2)
                        hg = (f16x2) { hu.x > (f16) 0 ? hu.x : (f16) 0, hu.y > (f16) 0 ? hu.y : (f16) 0 };
                    f16x2 uu = hu;
                    if (a.act_limit != 0.0f)
                    {
                        uu.x = uu.x < -lim ? -lim : (uu.x > lim ? lim : uu.x);
                        uu.y = uu.y < -lim ? -lim : (uu.y > lim ? lim : uu.y);
                        hg.x = hg.x > lim ? lim : hg.x;
                        hg.y = hg.y > lim ? lim : hg.y;
                    }
                    gg[q] = as_u32(hg * uu);               // fp16 gate product
                }
                unpack8(sd[bq], s);
                hmul4(gg, s);                              // fp16 down pre-scale
                to_f32(gg, f);
                fwht128_g16<true>(f, lane);
                #pragma unroll
                for (int i = 0; i < 8; ++i) f[i] *= R128;
                to_h(f, gg);
                const float cs = group_sum16(gg);
                if (c < chunks)
                {
                    *(u32x4*) (a.ti_g + idx) = (u32x4) { gg[0], gg[1], gg[2], gg[3] };
                    if (g == 0) a.ps_d[(size_t) r * chunks + c] = cs;
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------- output
__global__ __launch_bounds__(256)
void moes_out_kernel(MoesArgs a)
{
    // per wave: its 4 chunks (16 lanes x 8 values each) transposed so that atomic i of lane g
    // adds element 16 i + g: 64 contiguous bytes per group and instruction instead of 16 lines
    __shared__ __align__(16) float tr[4][4 * 128];
    const int lane = threadIdx.x & 63, g = lane & 15, sub = lane >> 4;
    float* trw = tr[threadIdx.x >> 6] + 128 * sub;
    const int chunks = a.H / 128;
    const int nw = gridDim.x * 4;
    for (int r = wave_id(); r < a.pool_rows; r += nw)
    {
        const int pos = a.rowinfo[3 * r];
        if (pos < 0) continue;                             // (uniform) rows past the pass
        const int e = a.rowinfo[3 * r + 1], j = a.rowinfo[3 * r + 2];
        const float rs = R128 * (float) as_h(a.weight_sorted[pos]);
        const uint16_t* svh_d = (const uint16_t*) a.d_svh[e];
        const int64_t token = a.token_sorted[pos];
        for (int c0 = 0; c0 < chunks; c0 += 4 * EW_B)
        {
            u32x4 yv[EW_B], sv[EW_B];
            #pragma unroll
            for (int bq = 0; bq < EW_B; ++bq)
            {
                const int col = 128 * min(c0 + 4 * bq + sub, chunks - 1) + 8 * g;
                yv[bq] = ld16(a.ts_g + (size_t) r * a.H + col);
                sv[bq] = ld16(svh_d + col);
            }
            #pragma unroll
            for (int bq = 0; bq < EW_B; ++bq)
            {
                const int c = c0 + 4 * bq + sub;
                const int col = 128 * min(c, chunks - 1) + 8 * g;
                uint32_t w[4], s[4];
                float f[8];
                unpack8(yv[bq], w);
                to_f32(w, f);
                fwht128_g16(f, lane);
                unpack8(sv[bq], s);
                #pragma unroll
                for (int q = 0; q < 4; ++q)
                {
                    const f16x2 svv = as_h2(s[q]);
                    f[2 * q] = (f[2 * q] * rs) * (float) svv.x;
                    f[2 * q + 1] = (f[2 * q + 1] * rs) * (float) svv.y;
                }
                if (a.scratch)
                {
                    if (c < chunks)
                    {
                        float* dst = a.scratch + (size_t) (a.fused_base[e] + j) * a.H + col;
                        *(f32x4*) dst = (f32x4) { f[0], f[1], f[2], f[3] };
                        *(f32x4*) (dst + 4) = (f32x4) { f[4], f[5], f[6], f[7] };
                    }
                }
                else
                {
                    #pragma unroll
                    for (int i = 0; i < 8; ++i) trw[8 * g + i] = f[i];
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                    if (c < chunks)
                    {
                        float* dst = a.out + (size_t) token * a.H + 128 * c + g;
                        #pragma unroll
                        for (int i = 0; i < 8; ++i) atomicAdd(dst + 16 * i, trw[16 * i + g]);
                    }
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                }
            }
        }
    }
}

// Token-major output (atomic-free): wave w takes tokens w, w + waves, ...; for each of the
// token's sorted positions whose row is in this pass (inv_row, confirmed by rowinfo) it adds
// that row's down output -- rotated, times the routing weight and svh, as the slot form computes
// it -- into fp32 registers, 8 four-chunk groups at a time, then adds the sum into out once.
// One writer per token and pass, and a fixed summation order.
constexpr int OUTT_G = 8;                 // 4-chunk groups held in registers per sweep

__global__ __launch_bounds__(256)
void moes_outt_kernel(MoesArgs a)
{
    const int lane = threadIdx.x & 63, g = lane & 15, sub = lane >> 4;
    const int chunks = a.H / 128, groups = (chunks + 3) / 4;
    const int nw = gridDim.x * 4;
    for (int tok = wave_id(); tok < a.bsz; tok += nw)
    {
        const int p0 = a.tok_start[tok], p1 = a.tok_start[tok + 1];
        if (p0 == p1) continue;
        for (int g0 = 0; g0 < groups; g0 += OUTT_G)
        {
            float acc[OUTT_G][8];
            #pragma unroll
            for (int q = 0; q < OUTT_G; ++q)
                #pragma unroll
                for (int i = 0; i < 8; ++i) acc[q][i] = 0.0f;
            bool any = false;
            for (int pi = p0; pi < p1; ++pi)
            {
                const int pos = a.tok_pos[pi];
                const int r = a.inv_row[pos];
                if (r < 0 || r >= a.pool_rows || a.rowinfo[3 * r] != pos) continue;   // (uniform) not in this pass
                any = true;
                const int e = a.rowinfo[3 * r + 1];
                const float rs = R128 * (float) as_h(a.weight_sorted[pos]);
                const uint16_t* svh_d = (const uint16_t*) a.d_svh[e];
                u32x4 yv[OUTT_G], sv[OUTT_G];
                #pragma unroll
                for (int q = 0; q < OUTT_G; ++q)
                {
                    const int col = 128 * min(4 * (g0 + q) + sub, chunks - 1) + 8 * g;
                    yv[q] = ld16(a.ts_g + (size_t) r * a.H + col);
                    sv[q] = ld16(svh_d + col);
                }
                #pragma unroll
                for (int q = 0; q < OUTT_G; ++q)
                {
                    uint32_t w[4], s[4];
                    float f[8];
                    unpack8(yv[q], w);
                    to_f32(w, f);
                    fwht128_g16(f, lane);
                    unpack8(sv[q], s);
                    #pragma unroll
                    for (int j = 0; j < 4; ++j)
                    {
                        const f16x2 svv = as_h2(s[j]);
                        acc[q][2 * j] += (f[2 * j] * rs) * (float) svv.x;
                        acc[q][2 * j + 1] += (f[2 * j + 1] * rs) * (float) svv.y;
                    }
                }
            }
            if (!any) continue;
            #pragma unroll
            for (int q = 0; q < OUTT_G; ++q)
            {
                const int c = 4 * (g0 + q) + sub;
                if (c >= chunks) continue;
                float* dst = a.out + (size_t) tok * a.H + 128 * c + 8 * g;
                const f32x4 o0 = *(const f32x4*) dst, o1 = *(const f32x4*) (dst + 4);
                *(f32x4*) dst = (f32x4) { o0.x + acc[q][0], o0.y + acc[q][1], o0.z + acc[q][2], o0.w + acc[q][3] };
                *(f32x4*) (dst + 4) = (f32x4) { o1.x + acc[q][4], o1.y + acc[q][5], o1.z + acc[q][6], o1.w + acc[q][7] };
            }
        }
    }
}

// ------------------------------------------------------------------------------- fixed-order gather
constexpr int GATHER_MAX_TOPK = 32;      // exl3_moe.cu:408 MOE_GATHER_MAX_TOPK

__global__ __launch_bounds__(256)
void moes_sum_kernel(MoesGatherArgs a)
{
    __shared__ int64_t slots[GATHER_MAX_TOPK];
    __shared__ float wts[GATHER_MAX_TOPK];
    __shared__ int nslots;
    const int token = blockIdx.x;
    const int t = threadIdx.x;
    if (t < a.topk)
    {
        const int64_t as = (int64_t) token * a.topk + t;
        const int64_t e = a.flat_expert[as];
        int64_t slot = -1;
        float wt = 1.0f;
        if (e >= 0 && e < a.num_experts)
        {
            const int64_t kind = a.slot_kind[e];
            if (kind)
            {
                const int64_t pos = a.inv_order[as];
                slot = a.slot_base[e] + (pos - a.expert_start[e]);
                if (kind == 2) wt = (float) as_h(a.weight_sorted[pos]);
            }
        }
        slots[t] = slot;
        wts[t] = wt;
    }
    __syncthreads();
    if (t == 0)
    {
        int n = 0;
        for (int k = 0; k < a.topk; ++k)
            if (slots[k] >= 0) { slots[n] = slots[k]; wts[n] = wts[k]; ++n; }
        nslots = n;
    }
    __syncthreads();
    const int n = nslots;
    if (n == 0) return;
    for (int col = t; col < a.H; col += blockDim.x)
    {
        float sum = 0.0f;
        for (int k = 0; k < n; ++k) sum = __builtin_fmaf(a.scratch[slots[k] * a.H + col], wts[k], sum);
        a.out[(int64_t) token * a.H + col] += sum;
    }
}

int grid_for(long jobs, int cus)
{
    const long want = (jobs + 15) / 16;
    const long cap = 8L * cus;
    return (int) std::max(1L, std::min(want, cap));
}

}  // namespace

int exl3k_moes_plan(const MoesArgs& a, int pass_row0, hipStream_t s)
{
    hipLaunchKernelGGL(moes_plan_kernel, dim3(1), dim3(PLAN_THREADS), 0, s, a, pass_row0);
    return (int) hipGetLastError();
}

static int rows_grid(int rows, int cus)
{
    return (int) std::max(1L, std::min((long) (rows + 3) / 4, 8L * cus));
}

int exl3k_moes_gather(const MoesArgs& a, int cus, hipStream_t s)
{
    hipLaunchKernelGGL(moes_gather_kernel, dim3(rows_grid(a.pool_rows, cus)), dim3(256), 0, s, a);
    return (int) hipGetLastError();
}

int exl3k_moes_act(const MoesArgs& a, int cus, hipStream_t s)
{
    hipLaunchKernelGGL(moes_act_kernel, dim3(rows_grid(a.pool_rows, cus)), dim3(256), 0, s, a);
    return (int) hipGetLastError();
}

size_t exl3k_moes_tokens_lds(int bsz, int num_assign)
{
    return ((size_t) bsz + (size_t) num_assign + PLAN_THREADS) * 4;
}

int exl3k_moes_tokens(const MoesArgs& a, hipStream_t s)
{
    const size_t lds = exl3k_moes_tokens_lds(a.bsz, a.num_assign);
    static bool attr = false;
    if (!attr)
    {
        (void) hipFuncSetAttribute((const void*) moes_tokens_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        attr = true;
    }
    hipLaunchKernelGGL(moes_tokens_kernel, dim3(1), dim3(PLAN_THREADS), lds, s, a);
    return (int) hipGetLastError();
}

int exl3k_moes_out(const MoesArgs& a, int cus, hipStream_t s)
{
    if (!a.scratch && a.tok_start)
    {
        hipLaunchKernelGGL(moes_outt_kernel, dim3(rows_grid(a.bsz, cus)), dim3(256), 0, s, a);
        return (int) hipGetLastError();
    }
    hipLaunchKernelGGL(moes_out_kernel, dim3(rows_grid(a.pool_rows, cus)), dim3(256), 0, s, a);
    return (int) hipGetLastError();
}

int exl3k_moes_sum(const MoesGatherArgs& a, hipStream_t s)
{
    hipLaunchKernelGGL(moes_sum_kernel, dim3(a.tokens), dim3(256), 0, s, a);
    return (int) hipGetLastError();
}
