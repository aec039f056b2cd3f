// Decode-shaped EXL3 GEMV for gfx950: C = had(had(A o suh) @ W_hat) o svh, m = 1..8.
//
// Semantics of exl3_gemv_kernel / exl3_gemm (quant/exl3_gemv_kernel.cuh:186-482), built
// for CDNA4 from rocprof measurements:
//
// Work split.  The weight is a sequence of "slices" (one 16-row k-slice of one 128-column
// output chunk: 8 tiles, 256*K contiguous bytes), ordered column-chunk-major.  Workgroup b
// streams the SB slices [b*SB, (b+1)*SB) of one chunk; its 4 waves take every 4th slice, so
// they read adjacent rows, and every wave runs one software-pipelined stream.  SB divides
// k/16, so a workgroup never straddles two chunks; it is chosen on the host for several
// resident waves per SIMD (one wave per SIMD issues VALU at half rate on gfx950).
//
// Reduction.  The 4 waves reduce through LDS.  A chunk owned by one workgroup (SB = k/16)
// finishes in place; otherwise each workgroup stores an fp32 partial to its slot and a second
// small kernel (gemv_finish) sums the slots in slot order -- deterministic -- and applies the
// output rotation and svh.  No atomics: on MI355X a device-scope atomic per workgroup costs
// 2.5-11 us per launch (measured), more than the kernel boundary.
//
// Input rotation.  Each workgroup computes had(x o suh) (fp32 butterfly, rounded to fp16 as
// the reference's A_had) only for the 128-row chunks its slices touch, into LDS, stored as
// duplicated pairs (x, x) so one v_dot2 consumes a decoded weight's two fp16 halves.
//
// Decode (per weight: extract the 16-bit window, x = s*A (+B), mask/xor, one v_dot2):
//   3INST / MCG: the weight is lo + hi of the masked word; v_dot2((x, x), (lo, hi)) adds
//   x*lo + x*hi in fp32 instead of first rounding lo + hi to fp16 (the reference's weight
//   differs from this by at most half an fp16 ulp; outputs stay far inside 2e-3).
//   MUL1: w = h * k_inv + bias with h = 1024 + bytesum (an exact small integer): the kernel
//   accumulates x*h and applies k_inv and bias * sum(x) per segment, in fp32.
// All ops are full-rate gfx950 VALU (no high-half-only writes, which issue at half rate).
//
// Compiled once per K (EXL3_INST_K) to keep build units small.
#include "exl3_common.cuh"
#include "exl3_gemv_core.cuh"
#include "exl3_kernels.h"
#include "exl3_xcd.cuh"

#ifndef EXL3_INST_K
#define EXL3_INST_K 4
#endif
#ifndef EXL3_GEMV_PRIO
#define EXL3_GEMV_PRIO 3
#endif
// 2 slices: measured on MI355X against 4 (and 1, 8) over the 32-layer Llama-3-8B sweep in a graph,
// interleaved runs: 2130-2205 GB/s against 2030-2070 (more loads in flight lengthened the stream
// of every launch)
#ifndef EXL3_GEMV_PF
#define EXL3_GEMV_PF 2
#endif

using namespace exl3;

namespace {

// Instrumented builds (-DEXL3_GEMV_TRACE): wave timestamps (s_memrealtime, 100 MHz) taken after
// `dep` is available, stored by lane 0 with a vector store.
#ifdef EXL3_GEMV_TRACE
#define GEMV_STAMP(g, slot_i, dep)                                                              \
    do {                                                                                        \
        uint64_t t_;                                                                            \
        asm volatile("s_memrealtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t_) : "s"(dep));        \
        if ((g).trace && (threadIdx.x & 63) == 0)          /* no trace buffer set: no stamp */  \
            (g).trace[(((size_t) blockIdx.y * gridDim.x + blockIdx.x) * 4 + (threadIdx.x >> 6)) * 8 + (slot_i)] = t_; \
    } while (0)
#else
#define GEMV_STAMP(g, slot_i, dep) do { } while (0)
#endif

constexpr int GEMV_THREADS = 256;
constexpr int GEMV_WAVES = 4;

// ---------------------------------------------------------------------------------------------
// Per-slot view of one launch (quant/exl3_gemm_kernel.cuh:169-238): slot j computes
// A[j or 0] @ B[q] with q = indices[j] (or j); table entries give the trellis, the input /
// output sign vectors, the width, the row stride (sliced mode: column slices of a wider
// matrix) and the output pointer.  Scalar loads only.
// ---------------------------------------------------------------------------------------------
struct MatView
{
    const uint16_t* A;
    const uint16_t* trellis;
    void* C;
    const uint16_t* suh;
    const uint16_t* svh;
    int n;          // this matrix's width
    int stride;     // row stride of trellis tiles (in columns) and of C
    float scale;    // output scale: 1/sqrt(128) (x routing weight)
};

// Scalar loads of the (uniform) table entries: issued together, one wait.  Absent tables are
// read at a harmless valid address (the kernel argument block's input pointer) and ignored.
__device__ __forceinline__ uint32_t s_load_u32(const void* p)
{
    uint32_t v;
    asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
    return v;
}

__device__ __forceinline__ bool resolve(const GemvArgs& g, int j, MatView& v)
{
    const size_t rows = g.slab_m ? g.slab_m : g.m;       // rows per slab
    const size_t elt = g.c_fp32 ? 4 : 2;
    int q = j;
    if (g.indices)
    {
        q = (int) s_load_u32(g.indices + j);      // low word of the int64 index (little endian)
        if (q < 0) return false;
    }
    const void* dummy = g.A;
    if (g.B_list)
    {
        const void* pB = g.B_list + q;
        const void* pV = g.svh_list + q;
        const void* pH = g.had_src ? (const void*) (g.had_src + q) : dummy;
        const void* pN = g.size_n ? (const void*) (g.size_n + q) : dummy;
        const void* pT = g.n_stride ? (const void*) (g.n_stride + q) : dummy;
        const void* pC = g.c_list ? (const void*) (g.c_list + q) : dummy;
        uint64_t b, vs, c;
        uint32_t h, nn, st;
        asm volatile("s_load_dwordx2 %0, %6, 0x0\n\t"
                     "s_load_dwordx2 %1, %7, 0x0\n\t"
                     "s_load_dword %2, %8, 0x0\n\t"
                     "s_load_dword %3, %9, 0x0\n\t"
                     "s_load_dword %4, %10, 0x0\n\t"
                     "s_load_dwordx2 %5, %11, 0x0\n\t"
                     "s_waitcnt lgkmcnt(0)"
                     : "=&s"(b), "=&s"(vs), "=&s"(h), "=&s"(nn), "=&s"(st), "=&s"(c)
                     : "s"(pB), "s"(pV), "s"(pH), "s"(pN), "s"(pT), "s"(pC)
                     : "memory");
        const int src = g.had_src ? (int) h : q;
        uint64_t u;
        asm volatile("s_load_dwordx2 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(u) : "s"(g.suh_list + src) : "memory");
        v.trellis = (const uint16_t*) b;
        v.svh = (const uint16_t*) vs;
        v.suh = (const uint16_t*) u;
        v.n = g.size_n ? (int) nn : g.n;
        v.stride = g.n_stride ? (int) st : v.n;
        if (g.c_list) v.C = (void*) c;
        else v.C = (char*) g.C + (size_t) j * rows * g.n * elt;
    }
    else
    {
        v.trellis = g.trellis;
        v.suh = g.suh;
        v.svh = g.svh;
        v.n = g.n;
        v.stride = g.n;
        v.C = (char*) g.C + (size_t) j * rows * g.n * elt;
    }
    // rows [row0, row0 + m) of the slab (row groups of a call with more than 8 rows)
    v.C = (char*) v.C + (size_t) g.row0 * v.stride * elt;
    v.A = g.A + (g.bszm_in == 1 ? (size_t) 0 : (size_t) j * rows * g.k) + (size_t) g.row0 * g.k;
    v.scale = EXL3_HAD_RSCALE;
    if (g.weights)
    {
        const uint32_t w2 = s_load_u32((const uint32_t*) ((uintptr_t) (g.weights + j) & ~(uintptr_t) 3));
        v.scale = EXL3_HAD_RSCALE * (float) as_h((uint16_t) ((j & 1) ? (w2 >> 16) : w2));
    }
    return true;
}

// Input rotation of chunks [kc0, kc0 + nkc) of rows [0, m) into xs (u32 units: 128
// duplicated pairs per chunk).  had_hf_r_128_inner<true,false> (hadamard_inner.cuh:93-150):
// fp16 pre-scale, fp32 butterfly, * 1/sqrt(128), round to fp16.
__device__ __forceinline__ void rotate_chunks(const uint16_t* __restrict__ A, const uint16_t* __restrict__ suh,
                                              uint32_t* xs, int xs_stride, int m, int k, int kc0, int nkc)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int job = wave; job < m * nkc; job += GEMV_WAVES)
    {
        const int row = job / nkc, c = job % nkc;
        const int col = (kc0 + c) * 128 + 2 * lane;
        f16x2 v = as_h2(*to_global((const uint32_t*) (A + (size_t) row * k + col)));
        f16x2 o;
        if (suh)
        {
            v = v * as_h2(*to_global((const uint32_t*) (suh + col)));
            float v0 = (float) v.x, v1 = (float) v.y;
            fwht128_wave(v0, v1, lane);
            o.x = (f16) (v0 * EXL3_HAD_RSCALE);
            o.y = (f16) (v1 * EXL3_HAD_RSCALE);
        }
        else o = v;
        f16x2 d0 = { o.x, o.x }, d1 = { o.y, o.y };
        u32x2 pr = { as_u32(d0), as_u32(d1) };
        *(u32x2*) (xs + row * xs_stride + c * 128 + 2 * lane) = pr;
    }
}

// Output rotation of one fp32 row chunk held as (v0, v1) = elements 2l, 2l+1, then store.
// Half output: had_fh_r_128_inner (hadamard_inner.cuh:216-281); float output: had_ff.
// `scale` is 1/sqrt(128), times the routing weight in weighted mode.
// svp: this lane's svh pair (svh[col], svh[col + 1]), loaded ahead by the caller.
__device__ __forceinline__ uint32_t store_output(float v0, float v1, void* C, int c_fp32, bool has_svh, uint32_t svp,
                                             size_t idx, int lane, float scale)
{
    if (has_svh)
    {
        fwht128_wave(v0, v1, lane);
        v0 *= scale;
        v1 *= scale;
        f16x2 s = as_h2(svp);
        if (!c_fp32)
        {
            f16x2 h = { (f16) v0, (f16) v1 };
            h = h * s;
            *to_global_w((uint32_t*) ((uint16_t*) C + idx)) = as_u32(h);
            return as_u32(h);
        }
        v0 *= (float) s.x;
        v1 *= (float) s.y;
    }
    if (c_fp32)
    {
        f32x2 o = { v0, v1 };
        *to_global_w((f32x2*) ((float*) C + idx)) = o;
        return 0u;
    }
    else
    {
        f16x2 h = { (f16) v0, (f16) v1 };
        *to_global_w((uint32_t*) ((uint16_t*) C + idx)) = as_u32(h);
        return as_u32(h);
    }
}

// Producer of a split residual norm (res_h non-null): fold the lane's stored fp16 output pair of
// row `row` into the residual stream and store the chunk's sum of squares.  Wave-level.
// hpre: the lane's h pair when the caller loaded it ahead (has_pre), else loaded here.
__device__ __forceinline__ void res_store(const GemvArgs& g, int row, int chunk, int lane, uint32_t cpair,
                                          bool has_pre = false, uint32_t hpre = 0u)
{
    if (!g.res_h) return;
    const size_t idx = (size_t) row * g.n + chunk * 128 + 2 * lane;
    const uint32_t hv = has_pre ? hpre : *to_global((const uint32_t*) (g.res_h + idx));
    const float t = res_pair_sq(hv, cpair, g.res_h, idx, lane);
    if (lane == 0) *to_global_w(g.res_sq + (size_t) row * (g.n / 128) + chunk) = t;
}

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

// Device-scope loads: they miss the CU's L1 and read the XCD's L2, where the other
// workgroups of the chunk (same XCD) left their results.
__device__ __forceinline__ f32x2 load_l2_f32x2(const float* p)
{
    return __builtin_bit_cast(f32x2, __hip_atomic_load(to_global((const uint64_t*) p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ uint32_t load_l2_u32(const void* p)
{
    return __hip_atomic_load(to_global((const uint32_t*) p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// All threads: release this workgroup's stores, count it in *ctr; true in the last arrival of
// `total` (which then re-arms the counter).
//
// Hardware assumption (outside the HIP memory model, which calls this a race between
// workgroups): every workgroup that counts in one counter runs on the same XCD, so its
// partial stores, the workgroup-scope atomic and the last arrival's L1-bypassing loads all
// meet in that XCD's L2, where gfx950 executes global atomics.  The host enables this mode
// only after exl3_device.hip's dispatch probe has shown, on this device, that workgroups b and
// b + xcd land on one XCD (round-robin dispatch); otherwise, and with EXL3_AMD_XCD=0, the
// partials are summed by the separate gemv_finish kernel.  Agent-scope atomics would not need
// the assumption but write back through the whole-device coherence point: 2.5-11 us per
// launch measured on MI355X.
__device__ __forceinline__ bool arrive_last(const XcdGuard& q, int* ctr, int total, int* flag)
{
    // the workgroup-scope release waits for LDS only: wait for this thread's global stores to be
    // acknowledged by the L2 before the counter can move
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __syncthreads();
    if (threadIdx.x == 0)
    {
        *flag = xcd_arrive(q, ctr, total);
    }
    __syncthreads();
    const bool last = *flag;
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    return last;
}

// Weighted reduction (quant/exl3_gemm_kernel.cuh:286-342) of the 128 columns of one chunk:
// token group t sums its bszm / num_tokens slots (ascending, inactive slots skipped) into
// output slab t, groups in increasing t.  fp16 outputs sum in fp16 like the reference.
__device__ void weighted_reduce(const GemvArgs& g, int chunk, bool via_l2)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int stride = g.bszm / g.num_tokens;
    // slabs hold all rows of the call; this launch owns rows [row0, row0 + m) of each
    const size_t slab = (size_t) (g.slab_m ? g.slab_m : g.m) * g.n;
    for (int t = 0; t < g.num_tokens; ++t)
    {
        for (int r = wave; r < g.m; r += GEMV_WAVES)
        {
            const size_t e = (size_t) (g.row0 + r) * g.n + chunk * 128 + 2 * lane;
            if (g.c_fp32)
            {
                float* C = (float*) g.C;
                float s0 = 0.0f, s1 = 0.0f;
                for (int jj = 0; jj < stride; ++jj)
                {
                    const int j = t * stride + jj;
                    if (g.indices && *to_global(g.indices + j) < 0) continue;
                    const float* p = C + (size_t) j * slab + e;
                    f32x2 v = via_l2 ? load_l2_f32x2(p) : *to_global((const f32x2*) p);
                    s0 += v.x; s1 += v.y;
                }
                f32x2 o = { s0, s1 };
                *to_global_w((f32x2*) (C + (size_t) t * slab + e)) = o;
            }
            else
            {
                uint16_t* C = (uint16_t*) g.C;
                f16x2 s = { (f16) 0.0f, (f16) 0.0f };
                for (int jj = 0; jj < stride; ++jj)
                {
                    const int j = t * stride + jj;
                    if (g.indices && *to_global(g.indices + j) < 0) continue;
                    const uint16_t* p = C + (size_t) j * slab + e;
                    s = s + as_h2(via_l2 ? load_l2_u32(p) : *to_global((const uint32_t*) p));
                }
                *to_global_w((uint32_t*) (C + (size_t) t * slab + e)) = as_u32(s);
            }
        }
        __syncthreads();   // group t + 1 may read slab t's rows written above by other waves
    }
}

// Block epilogue.  res: LDS [m][128] fp32, this workgroup's sums for its k range (all
// corrections applied).  One split: rotate and store.  Several splits: store the partial to
// this workgroup's slot; in XCD mode the last workgroup of the (slot j, chunk) pair then sums
// the partials -- in a fixed order -- rotates and stores.  Weighted mode adds a second hand-off
// per chunk over all slots, whose last arrival runs the token-group reduction.
__device__ void block_epilogue(const GemvArgs& g, const MatView& v, int j, int chunk, int slot, int splits,
                               const float* res, float* tmp, int* flag, uint32_t svp, int rs = 128)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m = g.m;
    const int chunks = g.n / 128;
    if (splits > 1)
    {
        float* pbase = g.partials + ((size_t) j * chunks + chunk) * splits * m * 128;
        for (int e = threadIdx.x; e < m * 32; e += GEMV_THREADS)
            *to_global_w((f32x4*) (pbase + (size_t) slot * m * 128 + 4 * e)) = *(const f32x4*) (res + (e >> 5) * rs + 4 * (e & 31));
        if (!g.xcd) return;
        GEMV_STAMP(g, 4, 0);
        if (!arrive_last(g.xg, g.counters + ((size_t) j * chunks + chunk) * 32, splits, flag)) return;
        GEMV_STAMP(g, 6, *flag);
        // sum the slots: threads split into G groups over the m * 64 column pairs; group gi takes
        // slots gi, gi + G, ...; the groups then combine in order through LDS
        const int pairs = m * 64;
        const int G = GEMV_THREADS / pairs > 0 ? GEMV_THREADS / pairs : 1;
        const int gi = threadIdx.x / pairs;
        const int pe = threadIdx.x % pairs;
        if (gi < G)
        {
            for (int pe2 = pe; pe2 < pairs; pe2 += GEMV_THREADS)
            {
                float s0 = 0.0f, s1 = 0.0f;
                for (int sp0 = gi; sp0 < splits; sp0 += 8 * G)
                {
                    f32x2 vv[8];
                    #pragma unroll
                    for (int u = 0; u < 8; ++u)
                        vv[u] = load_l2_f32x2(pbase + (size_t) min(sp0 + u * G, splits - 1) * m * 128 + 2 * pe2);
                    #pragma unroll
                    for (int u = 0; u < 8; ++u)
                        if (sp0 + u * G < splits) { s0 += vv[u].x; s1 += vv[u].y; }
                }
                tmp[(gi * pairs + pe2) * 2] = s0;
                tmp[(gi * pairs + pe2) * 2 + 1] = s1;
            }
        }
        __syncthreads();
        GEMV_STAMP(g, 7, 0);
        for (int r = wave; r < m; r += GEMV_WAVES)
        {
            float s0 = 0.0f, s1 = 0.0f;
            for (int q = 0; q < G; ++q)
            {
                s0 += tmp[(q * pairs + r * 64 + lane) * 2];
                s1 += tmp[(q * pairs + r * 64 + lane) * 2 + 1];
            }
            const int col = chunk * 128 + 2 * lane;
            res_store(g, r, chunk, lane,
                      store_output(s0, s1, v.C, g.c_fp32, v.svh != nullptr, svp, (size_t) r * v.stride + col, lane, v.scale));
        }
    }
    else
    {
        for (int r = wave; r < m; r += GEMV_WAVES)
        {
            const int col = chunk * 128 + 2 * lane;
            res_store(g, r, chunk, lane,
                      store_output(res[r * rs + 2 * lane], res[r * rs + 2 * lane + 1], v.C, g.c_fp32, v.svh != nullptr,
                                   svp, (size_t) r * v.stride + col, lane, v.scale));
        }
    }
    if (g.weights && g.xcd)
    {
        if (!arrive_last(g.xg, g.counters + g.counters_half + (size_t) chunk * 32, g.bszm, flag)) return;
        weighted_reduce(g, chunk, true);
    }
}

// Fused residual add + RMSNorm of the whole output row (rms_norm_res, amp_kernels.cu:279-365),
// run by the one wave that completes the row's last column chunk: h = fp16(h + C) in place,
// r = fp16(fp16(h * rsqrt(mean(h^2) + eps)) * w).  Lane l holds columns 8 l .. 8 l + 7 of each
// 512-column block; up to 8 blocks stay in registers between the two passes.
constexpr int NORM_RC = 8;

__device__ __noinline__ void fused_norm_wave(const uint16_t* C, uint16_t* h, const uint16_t* wn, uint16_t* rn,
                                             int n, float eps)
{
    const int lane = threadIdx.x & 63;
    float acc = 0.0f;
    u32x4 yk[NORM_RC];
    auto add_block = [&](int col, u32x4& out) {
        const u32x4 cv = *to_global((const u32x4*) (C + col));
        const u32x4 hv = *to_global((const u32x4*) (h + col));
        const uint32_t cw[4] = { cv.x, cv.y, cv.z, cv.w }, hw[4] = { hv.x, hv.y, hv.z, hv.w };
        uint32_t yw[4];
        #pragma unroll
        for (int q = 0; q < 4; ++q)
        {
            const f16x2 a = as_h2(hw[q]), b = as_h2(cw[q]);
            const f16x2 y = { (f16) ((float) a.x + (float) b.x), (f16) ((float) a.y + (float) b.y) };
            yw[q] = as_u32(y);
            acc += (float) y.x * (float) y.x + (float) y.y * (float) y.y;
        }
        out = (u32x4) { yw[0], yw[1], yw[2], yw[3] };
        *to_global_w((u32x4*) (h + col)) = out;
    };
    #pragma unroll
    for (int i = 0; i < NORM_RC; ++i)
    {
        const int col = 512 * i + 8 * lane;
        if (col < n) add_block(col, yk[i]);
    }
    for (int col = 512 * NORM_RC + 8 * lane; col < n; col += 512)
    {
        u32x4 t;
        add_block(col, t);
    }
    #pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
    const float scale = 1.0f / sqrtf(acc / (float) n + eps);
    auto norm_block = [&](int col, const u32x4& yv) {
        const u32x4 wv = *to_global((const u32x4*) (wn + col));
        const uint32_t yw[4] = { yv.x, yv.y, yv.z, yv.w }, ww[4] = { wv.x, wv.y, wv.z, wv.w };
        uint32_t o[4];
        #pragma unroll
        for (int q = 0; q < 4; ++q)
        {
            const f16x2 y = as_h2(yw[q]);
            o[q] = as_u32((f16x2) { (f16) ((float) y.x * scale), (f16) ((float) y.y * scale) } * as_h2(ww[q]));
        }
        *to_global_w((u32x4*) (rn + col)) = (u32x4) { o[0], o[1], o[2], o[3] };
    };
    #pragma unroll
    for (int i = 0; i < NORM_RC; ++i)
    {
        const int col = 512 * i + 8 * lane;
        if (col < n) norm_block(col, yk[i]);
    }
    for (int col = 512 * NORM_RC + 8 * lane; col < n; col += 512)
    {
        const u32x4 yv = *to_global((const u32x4*) (h + col));
        norm_block(col, yv);
    }
}

// Row completion for the fused norm: this wave has stored its chunk of C.  Release the stores at
// device scope (the row's chunks finish on every XCD), count the chunk; the last chunk's wave
// acquires and normalises the row, then re-arms the counter.  No wave ever waits on another.
__device__ __forceinline__ void norm_arrive(const GemvArgs& g, const uint16_t* C)
{
    const int lane = threadIdx.x & 63;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    int prev = 0;
    if (lane == 0) prev = __hip_atomic_fetch_add(to_global_w(g.norm_ctr), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = __builtin_amdgcn_readfirstlane(prev);
    if (prev != g.n / 128 - 1) return;
    if (lane == 0) __hip_atomic_store(to_global_w(g.norm_ctr), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    fused_norm_wave(C, g.norm_h, g.norm_w, g.norm_r, g.n, g.norm_eps);
}

// One wave's epilogue of an M = 1 chunk (no routing weights): v0, v1 are this workgroup's sums
// of columns 2 lane, 2 lane + 1 (corrections applied).  One split: rotate and store.  Several:
// store the partial to this workgroup's slot; in XCD mode count it in the chunk's counter (the
// wave waits for its stores first: the workgroup-scope release orders LDS only) and, in the last
// arrival, sum the slots in order, rotate and store.  Wave-level only: the workgroup's other
// waves have ended.
__device__ void finish_m1_wave(const GemvArgs& g, const MatView& v, int j, int chunk, int slot, int splits,
                               float v0, float v1, uint32_t svp, uint32_t hpre)
{
    const int lane = threadIdx.x & 63;
    const int col = chunk * 128 + 2 * lane;
    if (splits == 1)
    {
        res_store(g, 0, chunk, lane, store_output(v0, v1, v.C, g.c_fp32, v.svh != nullptr, svp, (size_t) col, lane, v.scale),
                  true, hpre);
        if (g.norm_h) norm_arrive(g, (const uint16_t*) v.C);
        return;
    }
    float* pbase = g.partials + ((size_t) j * (g.n / 128) + chunk) * splits * 128;
    *to_global_w((f32x2*) (pbase + (size_t) slot * 128 + 2 * lane)) = (f32x2) { v0, v1 };
    if (!g.xcd) return;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    int* ctr = g.counters + ((size_t) j * (g.n / 128) + chunk) * 32;
    int last = 0;
    if (lane == 0) last = xcd_arrive(g.xg, ctr, splits);
    if (!__builtin_amdgcn_readfirstlane(last)) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    // all slots' loads in flight together (16 per round: one L2 round trip for most shapes)
    float s0 = 0.0f, s1 = 0.0f;
    for (int p0 = 0; p0 < splits; p0 += 16)
    {
        f32x2 vv[16];
        #pragma unroll
        for (int u = 0; u < 16; ++u) vv[u] = load_l2_f32x2(pbase + (size_t) min(p0 + u, splits - 1) * 128 + 2 * lane);
        #pragma unroll
        for (int u = 0; u < 16; ++u)
            if (p0 + u < splits) { s0 += vv[u].x; s1 += vv[u].y; }
    }
    res_store(g, 0, chunk, lane, store_output(s0, s1, v.C, g.c_fp32, v.svh != nullptr, svp, (size_t) col, lane, v.scale),
              true, hpre);
    if (g.norm_h) norm_arrive(g, (const uint16_t*) v.C);
}

// Inactive slot (negative index) in weighted XCD mode: still counted once per chunk.
__device__ void inactive_arrive(const GemvArgs& g, int chunk, int slot, int* flag)
{
    if (!(g.weights && g.xcd) || slot != 0) return;
    if (!arrive_last(g.xg, g.counters + g.counters_half + (size_t) chunk * 32, g.bszm, flag)) return;
    weighted_reduce(g, chunk, true);
}

// Workgroup -> (chunk, split slot).  XCD mode: the splits of a chunk share one XCD.
__device__ __forceinline__ void block_coords(const GemvArgs& g, int splits, int& chunk, int& slot)
{
    gemv_block_coords(g.xcd, splits, (int) blockIdx.x, chunk, slot);
}

template <int K, int CB, int MT>
__global__ __launch_bounds__(GEMV_THREADS)
void gemv_kernel(const GemvArgs g)
{
    extern __shared__ __align__(16) uint32_t smem[];
    __shared__ int flag;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t a3 = sconst(89226354u), b3 = vconst(64248484u);       // 3INST multiplier, addend
    const int m = g.m, k = g.k;
    const int KS = k / 16;                                // slices per column chunk
    const int SB = g.slices_per_block;
    const int splits = KS / SB;
    const int j = blockIdx.y;
    int chunk, slot;
    block_coords(g, splits, chunk, slot);
    MatView v;
    if (!resolve(g, j, v)) { inactive_arrive(g, chunk, slot, &flag); return; }
    if (chunk * 128 >= v.n) return;
    // (unconditional load: without svh it reads the input, k >= 128, and is unused)
    const uint32_t svp = *to_global((const uint32_t*) ((v.svh ? v.svh + chunk * 128 : v.A) + 2 * lane));
    const int ks0 = slot * SB;
    const int kc0 = ks0 / 8;
    const int nkc = (ks0 + SB - 1) / 8 - kc0 + 1;
    const int xs_stride = g.xs_chunks * 128;              // u32 per row
    uint32_t* xs = smem;                                  // [MT][xs_chunks][128] dup pairs
    float* red = (float*) (smem + MT * xs_stride);        // [GEMV_WAVES][MT][128]

    // this wave's slices: ks0 + wave + 4 i, i < myn
    const int myn = SB > wave ? (SB - wave + GEMV_WAVES - 1) / GEMV_WAVES : 0;
    const int tiles_n = v.stride / 16;
    constexpr int KB = kbits(K);                          // whole words per lane (rate code K)
    const size_t kstride = (size_t) GEMV_WAVES * tiles_n * tile_words(K);   // u32 between my slices
    const uint32_t* base = (const uint32_t*) v.trellis + lane_word_off<K>(lane)
                         + ((size_t) (ks0 + min(wave, SB - 1)) * tiles_n + chunk * 8) * tile_words(K);

    // prefetch ring (unconditional, clamped loads keep the wait counts static)
    constexpr int PF = EXL3_GEMV_PF;
    const int last_i = myn > 0 ? myn - 1 : 0;
    const int prev_off = (lane & 7) == 0 ? 8 * K - 1 : -1;   // ring predecessor of my first word
    uint32_t ring[PF][KB + 1];
    #pragma unroll
    for (int d = 0; d < PF; ++d) load_slot_k<K>(base + (size_t) min(d, last_i) * kstride, prev_off, lane, ring[d]);

    // input rotation of the chunks this workgroup touches (overlaps the first loads)
    rotate_chunks(v.A, v.suh, xs, xs_stride, m, k, kc0, nkc);
    __syncthreads();

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
            const int ks = ks0 + wave + min(i, last_i) * GEMV_WAVES;
            const int xo = (ks / 8 - kc0) * 128 + (ks & 7) * 16;
            uint32_t wv[KB + 1];
            #pragma unroll
            for (int w = 0; w <= KB; ++w) wv[w] = ring[d][w];
            uint32_t raw[32];
            raw32<K, CB>(wv, raw, a3, b3);
            // refill this ring slot once its words are dead
            load_slot_k<K>(base + (size_t) min(i + PF, last_i) * kstride, prev_off, lane, ring[d]);

            #pragma unroll
            for (int r = 0; r < MT; ++r)
            {
                if (MT > 1 && r >= m) break;
                const u32x4* xp = (const u32x4*) (xs + r * xs_stride + xo);
                uint32_t x16[16];
                #pragma unroll
                for (int q = 0; q < 4; ++q)
                {
                    u32x4 t = xp[q];
                    x16[4 * q] = live ? t.x : 0u;     x16[4 * q + 1] = live ? t.y : 0u;
                    x16[4 * q + 2] = live ? t.z : 0u; x16[4 * q + 3] = live ? t.w : 0u;
                }
                // window w = 8g + jj: column j + 8 (jj >= 4), row 2g + {0, 1, 8, 9}[jj & 3]
                #pragma unroll
                for (int w = 0; w < 32; ++w)
                {
                    const int gq = w >> 3, jj = w & 7;
                    const int row = 2 * gq + (jj & 1) + 8 * ((jj >> 1) & 1);
                    float& a = acc[r][jj >> 2];
                    a = __builtin_amdgcn_fdot2(as_h2(x16[row]), as_h2(raw[w]), a, false);
                }
            }
        }
    }

    // cross-wave reduction; lane l of tile t owns columns 16t + (l & 7) and + 8
    const int c0 = (lane >> 3) * 16 + (lane & 7);
    #pragma unroll
    for (int r = 0; r < MT; ++r)
    {
        if (MT > 1 && r >= m) break;
        red[(wave * MT + r) * 128 + c0] = acc[r][0];
        red[(wave * MT + r) * 128 + c0 + 8] = acc[r][1];
    }
    __shared__ float sumx[8];
    if (CB == 2)
    {
        // MUL1 bias term: sum of the rotated input over this workgroup's k range
        for (int r = wave; r < m; r += GEMV_WAVES)
        {
            float sv = 0.0f;
            for (int e = lane; e < SB * 16; e += 64)
            {
                const int ks = ks0 + e / 16;
                sv += (float) as_h2(xs[r * xs_stride + (ks / 8 - kc0) * 128 + (ks & 7) * 16 + (e & 15)]).x;
            }
            sv = wave_sum(sv, lane);
            if (lane == 0) sumx[r] = sv;
        }
    }
    __syncthreads();

    // rows of the chunk -> res (LDS, reusing the input area): 4 waves x 64 lanes, two columns per lane
    float* res = (float*) xs;                             // [m][128]
    float r0[2][2];
    int nr = 0;
    for (int r = wave; r < m; r += GEMV_WAVES, ++nr)
    {
        const int c = 2 * lane;
        float v0 = red[r * 128 + c], v1 = red[r * 128 + c + 1];
        #pragma unroll
        for (int w = 1; w < GEMV_WAVES; ++w)
        {
            v0 += red[(w * MT + r) * 128 + c];
            v1 += red[(w * MT + r) * 128 + c + 1];
        }
        if (CB == 2)
        {
            const float kinv = (float) as_h(0x1eee), bias = sumx[r] * (float) as_h(0xc931);
            v0 = v0 * kinv + bias;
            v1 = v1 * kinv + bias;
        }
        r0[nr][0] = v0; r0[nr][1] = v1;
    }
    __syncthreads();                                      // xs reads done before res overwrites it
    nr = 0;
    for (int r = wave; r < m; r += GEMV_WAVES, ++nr)
    {
        res[r * 128 + 2 * lane] = r0[nr][0];
        res[r * 128 + 2 * lane + 1] = r0[nr][1];
    }
    __syncthreads();
    block_epilogue(g, v, j, chunk, slot, splits, res, red, &flag, svp);
}

// Sum the split partials of each (slot, column chunk) in slot order, output rotation, store.
// Grid: (n / 128, bszm); one wave per row.  Used when the XCD hand-off is off.
__global__ __launch_bounds__(GEMV_THREADS)
void gemv_finish(const GemvArgs g, int splits)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int chunk = blockIdx.x, j = blockIdx.y;
    MatView v;
    if (!resolve(g, j, v) || chunk * 128 >= v.n) return;
    const int m = g.m;
    const float* pbase = g.partials + ((size_t) j * (g.n / 128) + chunk) * splits * m * 128;
    for (int r = wave; r < m; r += GEMV_WAVES)
    {
        const int c = 2 * lane;
        const float* pp = pbase + (size_t) r * 128 + c;
        float v0 = 0.0f, v1 = 0.0f;
        for (int sp0 = 0; sp0 < splits; sp0 += 8)
        {
            f32x2 vv[8];
            #pragma unroll
            for (int u = 0; u < 8; ++u)
                vv[u] = __builtin_nontemporal_load(to_global((const f32x2*) (pp + (size_t) min(sp0 + u, splits - 1) * m * 128)));
            #pragma unroll
            for (int u = 0; u < 8; ++u)
                if (sp0 + u < splits) { v0 += vv[u].x; v1 += vv[u].y; }
        }
        const int col = chunk * 128 + c;
        const uint32_t svp = v.svh ? *to_global((const uint32_t*) (v.svh + col)) : 0u;
        res_store(g, r, chunk, lane,
                  store_output(v0, v1, v.C, g.c_fp32, v.svh != nullptr, svp, (size_t) r * v.stride + col, lane, v.scale));
    }
}

// Weighted reduction as its own kernel (XCD hand-off off).  Grid: n / 128.
__global__ __launch_bounds__(GEMV_THREADS)
void gemv_weighted_reduce(const GemvArgs g)
{
    weighted_reduce(g, blockIdx.x, false);
}

// ---------------------------------------------------------------------------------------------
// M = 1 streaming kernel.  Wave w of workgroup (chunk, slot) owns the W = SB/4 consecutive
// k-slices [ks0 + w W, ks0 + (w+1) W): W in {1, 2, 4} (part of one 128-row input chunk) or a
// multiple of 8 (whole chunks), so the waves run independently until the final reduction.
// Per input chunk the wave rotates x itself (lane l holds the rotated pair x[2l], x[2l+1] in
// one VGPR; the next chunk's x and suh are prefetched with the weights), and per k-slice eight
// v_readlane move that slice's 16 inputs to SGPRs, duplicated into (x, x) pairs by scalar
// packs; v_dot2 reads them there.  No LDS traffic and no barrier in the stream; every load is
// unconditional (clamped), so the compiler's wait counts stay exact and the PF-deep ring never
// drains.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t rotate_pair(uint32_t xv, uint32_t sv, bool has_suh, int lane)
{
    if (!has_suh) return xv;
    f16x2 v = as_h2(xv) * as_h2(sv);
    float v0 = (float) v.x, v1 = (float) v.y;
    fwht128_wave(v0, v1, lane);
    f16x2 o = { (f16) (v0 * EXL3_HAD_RSCALE), (f16) (v1 * EXL3_HAD_RSCALE) };
    return as_u32(o);
}

// Fused SwiGLU input (IN = GEMV_IN_SILU): the pair of silu(gate) * up, rounded to fp16 as silu_mul does.
__device__ __forceinline__ uint32_t silu_mul_pair(uint32_t gv, uint32_t uv)
{
    const f16x2 gh = as_h2(gv), uh = as_h2(uv);
    const f16x2 o = { (f16) (silu_f32((float) gh.x) * (float) uh.x), (f16) (silu_f32((float) gh.y) * (float) uh.y) };
    return as_u32(o);
}

// Input forms (IN): 0 the input itself; 1 the fused SwiGLU pair (A = gate, A_up = up); 2 the
// consumer half of a split residual norm (A = the residual stream h, norm weights in_w, chunk
// sums of squares in_sq): every wave forms the scale itself, from the same sums in the same order.
enum { GEMV_IN_PLAIN = 0, GEMV_IN_SILU = 1, GEMV_IN_NORM = 2 };

template <int K, int CB, int WS, int IN>
__global__ __launch_bounds__(GEMV_THREADS)
// the split-norm input form asks for 4 waves per SIMD (at most 128 registers: left alone it takes
// 109 VGPRs + 24 AGPRs and runs 3 waves per SIMD, 21 -> 24 us on the stacked gate / up launch);
// the other forms keep their own allocation
__attribute__((amdgpu_waves_per_eu(IN == 2 ? 4 : 1)))
void gemv1_kernel(const GemvArgs g)
{
    __shared__ __align__(16) float red[GEMV_WAVES][128];
    __shared__ __align__(16) float res[128];
    __shared__ __align__(16) float tmp[2 * GEMV_THREADS];
    __shared__ float sumx_w[GEMV_WAVES];
    __shared__ int flag;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t a3 = sconst(89226354u), b3 = vconst(64248484u);       // 3INST multiplier, addend
    const int KS = g.k / 16;
    const int SB = g.slices_per_block;
    const int splits = KS / SB;
    const int j = blockIdx.y;
    int chunk, slot;
    block_coords(g, splits, chunk, slot);
    MatView v;
    if (!resolve(g, j, v)) { inactive_arrive(g, chunk, slot, &flag); return; }
    if (chunk * 128 >= v.n) return;
    // Wave priority: a wave that starts (input load and rotation) or ends (hand-off) outranks
    // the waves in their decode loops, so that no wave of the SIMD is starved at either end of
    // its stream while older waves keep the VALU busy
    __builtin_amdgcn_s_setprio(EXL3_GEMV_PRIO);
#ifdef EXL3_GEMV_TRACE
    {
        uint32_t hw, xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)\n\ts_getreg_b32 %1, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(hw), "=s"(xcc));
        GEMV_STAMP(g, 0, hw);
        if (g.trace && (threadIdx.x & 63) == 0)
            g.trace[(((size_t) blockIdx.y * gridDim.x + blockIdx.x) * 4 + (threadIdx.x >> 6)) * 8 + 5] = ((uint64_t) xcc << 32) | hw;
    }
#endif

    // WS: slices per wave when below 8 (W = WS), else 8 (W a multiple of 8)
    const int W = SB / GEMV_WAVES;
    const int a = slot * SB + wave * W;                 // first k-slice of this wave
    const int nchunks = WS < 8 ? 1 : W / 8;
    __builtin_assume(nchunks >= 1);                     // the planner's W is 1, 2, 4 or a multiple of 8
    constexpr int per = WS;                             // slices per input chunk
    const int lane0 = WS < 8 ? (a & 7) * 8 : 0;         // x lanes of the first slice
    const int tiles_n = v.stride / 16;
    constexpr int KB = kbits(K);                        // whole words per lane (rate code K)
    const size_t rstride = (size_t) tiles_n * tile_words(K);    // u32 per k-slice row
    const uint32_t* base = (const uint32_t*) v.trellis + lane_word_off<K>(lane)
                         + ((size_t) a * tiles_n + chunk * 8) * tile_words(K);
    const int prev_off = (lane & 7) == 0 ? 8 * K - 1 : -1;
    const uint32_t* sinkp = g.sink + 64 + lane_word_off<K>(lane);      // +64: room for prev_off = -1
    const bool has_suh = v.suh != nullptr;
    const uint32_t* xg = (const uint32_t*) v.A + lane;                       // x pairs
    const uint32_t* sg = (const uint32_t*) (has_suh ? v.suh : v.A) + lane;   // suh pairs
    // up pairs (fused SwiGLU) or norm weight pairs (split norm)
    const uint32_t* ug = (const uint32_t*) (IN == GEMV_IN_SILU ? g.A_up : IN == GEMV_IN_NORM ? g.in_w : v.A) + lane;

    constexpr int PF = EXL3_GEMV_PF;
    static_assert(8 % PF == 0, "prefetch depth must divide 8");
    const int last = W - 1;
    // x of the first chunk first (its wait then leaves the weight loads in flight).  The input,
    // suh and up vectors are read by every wave: cached loads, so that they stay in the XCD's
    // L2 after the first miss (nontemporal loads made every wave's read queue behind the weight
    // stream in HBM: 3-12 us before the first dot, measured with per-wave timestamps)
    uint32_t xv = *(to_global(xg) + (size_t) (a / 8) * 64);
    uint32_t sv = *(to_global(sg) + (size_t) (a / 8) * 64);
    uint32_t uv = 0u;
    if constexpr (IN != GEMV_IN_PLAIN) uv = *(to_global(ug) + (size_t) (a / 8) * 64);
    // split norm: the chunk sums with the inputs; the scale is formed once the weights are in flight
    float sqv[SQ_SCALE_MAX_PER_LANE];
    if constexpr (IN == GEMV_IN_NORM) sq_load(g.in_sq, g.k / 128, lane, sqv);
    // keep them ahead of the weight loads: loads return in issue order, so an input load the
    // scheduler moved behind the ring would wait for the ring's slices
    __builtin_amdgcn_sched_barrier(0);
    uint32_t ring[PF][KB + 1];
    #pragma unroll
    for (int d = 0; d < PF; ++d) load_slot_k<K>(base + (size_t) min(d, last) * rstride, prev_off, lane, ring[d]);
    // svh pair for the epilogue, behind the first weights
    // (unconditional load: without svh it reads the input, k >= 128, and is unused)
    const uint32_t svp = *to_global((const uint32_t*) ((v.svh ? v.svh + chunk * 128 : v.A) + 2 * lane));
    // the residual pair for a split norm's producer epilogue (unconditional as svp)
    const uint32_t hpre = *to_global((const uint32_t*) ((g.res_h ? g.res_h + chunk * 128 : v.A) + 2 * lane));
    float nscale = 0.0f;
    if constexpr (IN == GEMV_IN_NORM) nscale = sq_scale(sqv, g.k, g.in_eps, lane);

    float sx = 0.0f;
    // Dot products on the matrix pipe, v_mfma_f32_16x16x32_f16: lane l's A operand is 4 k rows
    // of one of its columns as decoded (lo, hi) fp16 pairs; B is block-diagonal over the four
    // 16-lane groups (lane 16 q + n holds the rows' (x, x) pairs iff n == q, zeros otherwise), so
    // the 32-long dot of row r, column n is lane 16 n + r's own 8 products: D[r][n] accumulates
    // lane 16 n + r's dot.  The x pairs come from LDS (the off-diagonal lanes read a zero region
    // at the same offsets).  The matrix pipe runs beside the other waves' decode VALU; the
    // 4x4x4 form this replaces issued like VALU (measured gate/up 23.1 -> 22.2 us).
    __shared__ __align__(16) uint32_t xdup[GEMV_WAVES][2][128];
    __shared__ __align__(16) uint32_t xzero[GEMV_WAVES][128];
    *(u32x2*) &xzero[wave][2 * lane] = (u32x2) { 0u, 0u };
    const bool diag = (lane & 15) == (lane >> 4);
    f32x4 accv[4] = { { 0, 0, 0, 0 }, { 0, 0, 0, 0 }, { 0, 0, 0, 0 }, { 0, 0, 0, 0 } };
    for (int c = 0; c < nchunks; ++c)
    {
        const uint32_t xi = IN == GEMV_IN_SILU ? silu_mul_pair(xv, uv) : IN == GEMV_IN_NORM ? norm_pair(xv, uv, nscale) : xv;
        const uint32_t xr = rotate_pair(xi, sv, has_suh, lane);
        if (c == 0) GEMV_STAMP(g, 1, __builtin_amdgcn_readfirstlane(xr));
        if (c == 0) __builtin_amdgcn_s_setprio(0);
        if (CB == 2)
        {
            const f16x2 p = as_h2(xr);
            const bool mine = WS == 8 || (lane >= lane0 && lane < lane0 + 8 * per);
            sx += wave_sum(mine ? (float) p.x + (float) p.y : 0.0f, lane);
        }
        uint32_t* xd = xdup[wave][c & 1];
        {
            // rows 2 lane, 2 lane + 1 of the chunk at slice position 4 g + 2 h + e for slice row
            // t = 2 g + e + 8 h: each B operand is 4 contiguous words
            const f16x2 p = as_h2(xr);
            const f16x2 d0 = { p.x, p.x }, d1 = { p.y, p.y };
            const int t = (2 * lane) & 15;
            *(u32x2*) (xd + ((2 * lane) & ~15) + 4 * ((t & 7) >> 1) + 2 * (t >> 3)) = (u32x2) { as_u32(d0), as_u32(d1) };
        }
        const uint32_t* bbase = diag ? xd + (lane0 / 8) * 16 : xzero[wave];
        __builtin_amdgcn_wave_barrier();
        // prefetch the next chunk's x (clamped: stays inside this wave's range)
        const int cn = min(c + 1, nchunks - 1);
        xv = *(to_global(xg) + (size_t) (a / 8 + cn) * 64);
        sv = *(to_global(sg) + (size_t) (a / 8 + cn) * 64);
        if constexpr (IN != GEMV_IN_PLAIN) uv = *(to_global(ug) + (size_t) (a / 8 + cn) * 64);
        #pragma unroll
        for (int s8 = 0; s8 < per; ++s8)
        {
            const int i = c * 8 + s8;
            const int d = s8 % PF;
            uint32_t wv[KB + 1];
            #pragma unroll
            for (int w = 0; w <= KB; ++w) wv[w] = ring[d][w];
            // refill with slice i + PF; past the last slice it reads the 8 KiB sink, which every
            // wave's tail reads and nothing writes (L2-resident: no HBM traffic, and the hand-off's
            // wait for the partial stores does not wait on HBM).  Unconditional, so the wait
            // counts stay static.
            load_slot_k<K>(i + PF <= last ? base + (size_t) (i + PF) * rstride : sinkp, prev_off, lane, ring[d]);
            // decode per group of 8 windows, right before its 2 MFMAs: 8 live words instead of 32
            #pragma unroll
            for (int gq = 0; gq < 4; ++gq)
            {
                uint32_t raw[32];
                if (gq == 0) raw8<K, CB, 0>(wv, raw, a3, b3);
                else if (gq == 1) raw8<K, CB, 8>(wv, raw, a3, b3);
                else if (gq == 2) raw8<K, CB, 16>(wv, raw, a3, b3);
                else raw8<K, CB, 24>(wv, raw, a3, b3);
                const f16x8 bx = __builtin_bit_cast(f16x8, *(const u32x4*) (bbase + s8 * 16 + 4 * gq));
                #pragma unroll
                for (int cc = 0; cc < 2; ++cc)
                {
                    // windows 8 gq + 4 cc + (0..3): column cc, rows 2 gq, 2 gq + 1, 2 gq + 8, 2 gq + 9
                    const int w = 8 * gq + 4 * cc;
                    const u32x4 aw = { raw[w], raw[w + 1], raw[w + 2], raw[w + 3] };
                    accv[2 * (gq & 1) + cc] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        __builtin_bit_cast(f16x8, aw), bx, accv[2 * (gq & 1) + cc], 0, 0, 0);
                }
            }
        }
    }
    GEMV_STAMP(g, 2, __builtin_amdgcn_readfirstlane(__float_as_uint(accv[0].x)));
    __builtin_amdgcn_s_setprio(EXL3_GEMV_PRIO);
    {
        // lane L holds D[4 (L / 16) + i][L % 16]; for n = L % 16 < 4 that is the dot of lane
        // o = 16 n + 4 (L / 16) + i, whose columns are (o / 8) 16 + o % 8 (+ 8 for cc = 1)
        const int n = lane & 15;
        if (n < 4)
        {
            const f32x4 s0 = accv[0] + accv[2], s1 = accv[1] + accv[3];
            #pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                const int o = 16 * n + 4 * (lane >> 4) + i;
                const int co = (o >> 3) * 16 + (o & 7);
                red[wave][co] = s0[i];
                red[wave][co + 8] = s1[i];
            }
        }
    }
    if (lane == 0) sumx_w[wave] = sx;
    __syncthreads();
    if (!g.weights)
    {
        // one wave finishes the chunk; the other three end here, so their registers take the
        // next workgroups' waves instead of idling through the hand-off
        if (wave != 0) return;
        float v0 = red[0][2 * lane] + red[1][2 * lane] + red[2][2 * lane] + red[3][2 * lane];
        float v1 = red[0][2 * lane + 1] + red[1][2 * lane + 1] + red[2][2 * lane + 1] + red[3][2 * lane + 1];
        if (CB == 2)
        {
            const float kinv = (float) as_h(0x1eee);
            const float bias = (sumx_w[0] + sumx_w[1] + sumx_w[2] + sumx_w[3]) * (float) as_h(0xc931);
            v0 = v0 * kinv + bias;
            v1 = v1 * kinv + bias;
        }
        finish_m1_wave(g, v, j, chunk, slot, splits, v0, v1, svp, hpre);
        GEMV_STAMP(g, 3, 0);
        return;
    }
    if (threadIdx.x < 128)
    {
        const int c = threadIdx.x;
        float vv = red[0][c] + red[1][c] + red[2][c] + red[3][c];
        if (CB == 2)
        {
            const float kinv = (float) as_h(0x1eee);
            const float bias = (sumx_w[0] + sumx_w[1] + sumx_w[2] + sumx_w[3]) * (float) as_h(0xc931);
            vv = vv * kinv + bias;
        }
        res[c] = vv;
    }
    __syncthreads();
    block_epilogue(g, v, j, chunk, slot, splits, res, tmp, &flag, svp);
    GEMV_STAMP(g, 3, flag);
}

// ---------------------------------------------------------------------------------------------
// Balanced M = 1 stream (gemv1b_kernel).  gemv1_kernel gives every workgroup the same work, so a
// launch whose workgroup count is not a multiple of the resident capacity (the stacked gate / up
// bundle: 896 workgroups on 256 CUs, 3 or 4 waves per SIMD) leaves a quarter to a half of the
// SIMDs idle for the last third of the launch (per-wave timestamps on MI355X: loop ends from 8
// to 22 us).  Here every wave of the grid streams exactly R slices, and the grid is sized to put
// the same number of waves on every SIMD.
//
// Work order.  Column chunks of all matrices form pairs p = j * chunks + chunk; the pairs of XCD
// residue x (p % xcd == x) are concatenated, KS slices each.  Workgroup b (residue x = b % xcd,
// local index lb = b / xcd) takes slices [4 R lb, 4 R lb + 4 R) of that list, wave w the R slices
// from 4 R lb + w R.  4 R <= KS, so a workgroup's range covers the tail of one pair (A) and the
// head of the next (B) at most.  The four waves' sums meet in LDS per pair; the workgroup stores
// one partial of 128 fp32 per pair into slot lb - first(pair) and counts itself in the pair's
// counter; the last arrival (same XCD: the hand-off of finish_m1_wave) sums the pair's slots in
// slot order, rotates, scales by svh and stores.  Decode, prefetch ring and the 4x4x4
// matrix-core dot are gemv1_kernel's.
template <int K, int CB>
__global__ __launch_bounds__(GEMV_THREADS)
__attribute__((amdgpu_waves_per_eu(4, 4)))             // 4 waves per SIMD: at most 128 registers
void gemv1b_kernel(const GemvArgs g)
{
    __shared__ __align__(16) uint32_t xdup[GEMV_WAVES][2][128];
    __shared__ __align__(16) float red[2][GEMV_WAVES][128];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t a3 = sconst(89226354u), b3 = vconst(64248484u);
    const int KS = g.k / 16, R = g.slices_per_block, chunks = g.n / 128;
    const int X = g.xcd, lb = blockIdx.x / X;
    Gemv1bBlock blk;
    if (!gemv1b_block(X, g.bszm * chunks, KS, R, (int) blockIdx.x, blk)) return;
    const int T0 = lb * GEMV_WAVES * R;                   // the workgroup's first slice
    const int qA = blk.qA, Bd = (qA + 1) * KS;            // pair A and the first slice of pair B
    const bool straddle = blk.straddle;
    const int t0 = T0 + wave * R;
    const int n0 = min(max(Bd - t0, 0), R);               // this wave's slices in pair A
    const int sA0 = t0 - qA * KS, sB0 = t0 - Bd;          // slice i: A at sA0 + i, B at sB0 + i
    __builtin_amdgcn_s_setprio(EXL3_GEMV_PRIO);
#ifdef EXL3_GEMV_TRACE
    {
        uint32_t hw, xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)\n\ts_getreg_b32 %1, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(hw), "=s"(xcc));
        GEMV_STAMP(g, 0, hw);
        if (g.trace && (threadIdx.x & 63) == 0)
            g.trace[(((size_t) blockIdx.y * gridDim.x + blockIdx.x) * 4 + (threadIdx.x >> 6)) * 8 + 5] = ((uint64_t) xcc << 32) | hw;
    }
#endif

    // the two pairs' matrices (every field selected by a uniform condition: indexed arrays of
    // views would live in scratch)
    MatView va, vb;
    const int pa = blk.pa, pb = blk.pb;
    const int ja = pa / chunks, jb = pb / chunks;
    const int cha = pa - ja * chunks, chb = pb - jb * chunks;
    resolve(g, ja, va);
    resolve(g, jb, vb);
    const int tiles_n = va.stride / 16;
    const size_t rstride = (size_t) tiles_n * tile_words(K);
    const uint32_t lofs = lane_word_off<K>(lane);
    const uint32_t* baseA = (const uint32_t*) va.trellis + (size_t) cha * 8 * tile_words(K);
    const uint32_t* baseB = (const uint32_t*) vb.trellis + (size_t) chb * 8 * tile_words(K);
    const int prev_off = (lane & 7) == 0 ? 8 * K - 1 : -1;
    const bool has_suh = va.suh != nullptr;
    auto addr = [&](int i) {
        return (i < n0 ? baseA + (size_t) (sA0 + i) * rstride : baseB + (size_t) (sB0 + i) * rstride) + lofs;
    };
    // input pair of slice i's 128-row chunk (pair A or B's input and suh)
    auto xload = [&](int i, uint32_t& xv, uint32_t& sv) {
        const bool sb = i >= n0;
        const int sl = sb ? sB0 + i : sA0 + i;
        const uint16_t* A = sb ? vb.A : va.A;
        const uint16_t* su = has_suh ? (sb ? vb.suh : va.suh) : A;
        xv = *(to_global((const uint32_t*) A + lane) + (size_t) (sl >> 3) * 64);
        sv = *(to_global((const uint32_t*) su + lane) + (size_t) (sl >> 3) * 64);
    };
    // first slice of the input chunk after slice i's (a pair change starts a new chunk)
    auto next_group = [&](int i) {
        const int sl = i < n0 ? sA0 + i : sB0 + i;
        const int e = i + 8 - (sl & 7);
        return i < n0 ? min(e, n0) : e;
    };

    uint32_t xv, sv, xvn = 0u, svn = 0u;
    xload(0, xv, sv);
    int gnext = next_group(0);
    __builtin_amdgcn_sched_barrier(0);
    constexpr int KB = kbits(K);
    constexpr int PF = EXL3_GEMV_PF;
    uint32_t ring[PF][KB + 1];
    #pragma unroll
    for (int d = 0; d < PF; ++d) load_slot_k<K>(addr(min(d, R - 1)), prev_off, lane, ring[d]);
    if (gnext < R) xload(gnext, xvn, svn);

    // 16x16x32 dot with block-diagonal B, as in gemv1_kernel
    __shared__ __align__(16) uint32_t xzero[GEMV_WAVES][128];
    *(u32x2*) &xzero[wave][2 * lane] = (u32x2) { 0u, 0u };
    const bool diag = (lane & 15) == (lane >> 4);
    f32x4 accv[4] = { { 0, 0, 0, 0 }, { 0, 0, 0, 0 }, { 0, 0, 0, 0 }, { 0, 0, 0, 0 } };
    int xb = 0;
    const uint32_t* bbase = xzero[wave];
    // this wave's sums of one pair into red[sg][wave] (columns), or zeros: lane L holds the dots
    // of lanes o = 16 n + 4 (L / 16) + i (n = L % 16 < 4), columns (o / 8) 16 + o % 8 (+ 8)
    auto deposit = [&](int sg, bool zero) {
        const int n = lane & 15;
        if (n < 4)
        {
            const f32x4 s0 = accv[0] + accv[2], s1 = accv[1] + accv[3];
            #pragma unroll
            for (int i = 0; i < 4; ++i)
            {
                const int o = 16 * n + 4 * (lane >> 4) + i;
                const int co = (o >> 3) * 16 + (o & 7);
                red[sg][wave][co] = zero ? 0.0f : s0[i];
                red[sg][wave][co + 8] = zero ? 0.0f : s1[i];
            }
        }
    };

    for (int i0 = 0; i0 < R; i0 += PF)
    {
        #pragma unroll
        for (int d = 0; d < PF; ++d)
        {
            const int i = i0 + d;
            if (i >= R) break;
            if (i == n0 && n0 > 0)                        // pair A done: its sums to LDS, restart
            {
                deposit(0, false);
                #pragma unroll
                for (int a = 0; a < 4; ++a) accv[a] = (f32x4) { 0, 0, 0, 0 };
            }
            if (i == 0 || i == gnext)
            {
                if (i != 0) { xv = xvn; sv = svn; gnext = next_group(i); if (gnext < R) xload(gnext, xvn, svn); }
                const uint32_t xr = rotate_pair(xv, sv, has_suh, lane);
                if (i == 0) GEMV_STAMP(g, 1, __builtin_amdgcn_readfirstlane(xr));
                if (i == 0) __builtin_amdgcn_s_setprio(0);
                xb ^= 1;
                const f16x2 pq = as_h2(xr);
                const f16x2 d0 = { pq.x, pq.x }, d1 = { pq.y, pq.y };
                const int t = (2 * lane) & 15;
                *(u32x2*) (&xdup[wave][xb][((2 * lane) & ~15) + 4 * ((t & 7) >> 1) + 2 * (t >> 3)]) =
                    (u32x2) { as_u32(d0), as_u32(d1) };
                bbase = diag ? xdup[wave][xb] : xzero[wave];
                __builtin_amdgcn_wave_barrier();
            }
            const int xrow = ((i < n0 ? sA0 + i : sB0 + i) & 7) * 16;
            uint32_t wv[KB + 1];
            #pragma unroll
            for (int w = 0; w <= KB; ++w) wv[w] = ring[d][w];
            // past the last slice: the last slice again (just read, an L2 hit), so that the load
            // is unconditional and the wait counts stay static
            load_slot_k<K>(addr(min(i + PF, R - 1)), prev_off, lane, ring[d]);
            #pragma unroll
            for (int gq = 0; gq < 4; ++gq)
            {
                uint32_t raw[32];
                if (gq == 0) raw8<K, CB, 0>(wv, raw, a3, b3);
                else if (gq == 1) raw8<K, CB, 8>(wv, raw, a3, b3);
                else if (gq == 2) raw8<K, CB, 16>(wv, raw, a3, b3);
                else raw8<K, CB, 24>(wv, raw, a3, b3);
                const f16x8 bx = __builtin_bit_cast(f16x8, *(const u32x4*) (bbase + xrow + 4 * gq));
                #pragma unroll
                for (int cc = 0; cc < 2; ++cc)
                {
                    const int w = 8 * gq + 4 * cc;
                    const u32x4 aw = { raw[w], raw[w + 1], raw[w + 2], raw[w + 3] };
                    accv[2 * (gq & 1) + cc] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        __builtin_bit_cast(f16x8, aw), bx, accv[2 * (gq & 1) + cc], 0, 0, 0);
                }
            }
        }
    }
    GEMV_STAMP(g, 2, __builtin_amdgcn_readfirstlane(__float_as_uint(accv[0].x)));
    __builtin_amdgcn_s_setprio(EXL3_GEMV_PRIO);
    if (n0 == R) deposit(0, false);                       // all in pair A
    else deposit(1, false);                               // the rest is in pair B
    if (n0 == 0) deposit(0, true);                        // no slices of pair A
    if (straddle && n0 == R) deposit(1, true);            // no slices of pair B
    __syncthreads();

    // wave 0 finishes pair A, wave 1 pair B (when the workgroup straddles); the others end
    const bool sg = wave == 1;
    if (wave > 1 || (sg && !straddle)) return;
    const float v0 = red[sg][0][2 * lane] + red[sg][1][2 * lane] + red[sg][2][2 * lane] + red[sg][3][2 * lane];
    const float v1 = red[sg][0][2 * lane + 1] + red[sg][1][2 * lane + 1] + red[sg][2][2 * lane + 1] + red[sg][3][2 * lane + 1];
    const int q = qA + (sg ? 1 : 0);
    int first, n;
    gemv1b_pair_span(KS, R, q, first, n);
    void* Cp = sg ? vb.C : va.C;
    const uint16_t* svh = sg ? vb.svh : va.svh;
    const float scale = sg ? vb.scale : va.scale;
    const int pp = sg ? pb : pa;
    const int col = (sg ? chb : cha) * 128 + 2 * lane;
    const uint32_t svp = svh ? *to_global((const uint32_t*) (svh + col)) : 0u;
    if (n == 1)
    {
        store_output(v0, v1, Cp, g.c_fp32, svh != nullptr, svp, (size_t) col, lane, scale);
        return;
    }
    float* pbase = g.partials + (size_t) pp * g.slots * 128;
    *to_global_w((f32x2*) (pbase + (size_t) (lb - first) * 128 + 2 * lane)) = (f32x2) { v0, v1 };
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    int* ctr = g.counters + (size_t) pp * 32;
    int last = 0;
    if (lane == 0) last = xcd_arrive(g.xg, ctr, n);
    if (!__builtin_amdgcn_readfirstlane(last)) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    float a0 = 0.0f, a1 = 0.0f;
    for (int p0 = 0; p0 < n; p0 += 16)
    {
        f32x2 pv[16];
        #pragma unroll
        for (int u = 0; u < 16; ++u) pv[u] = load_l2_f32x2(pbase + (size_t) min(p0 + u, n - 1) * 128 + 2 * lane);
        #pragma unroll
        for (int u = 0; u < 16; ++u)
            if (p0 + u < n) { a0 += pv[u].x; a1 += pv[u].y; }
    }
    store_output(a0, a1, Cp, g.c_fp32, svh != nullptr, svp, (size_t) col, lane, scale);
    GEMV_STAMP(g, 3, 0);
}

// ---------------------------------------------------------------------------------------------
// Row-batched GEMV on the matrix cores (m = 1..16 rows per launch; the decode path uses it for
// m >= 2).  v_mfma_f32_16x16x32_f16 with
//   A (16 x 32): 16 output columns x 16 k-rows of the weight, each weight as its two fp16
//                halves (lo, hi) -- the 3INST / MCG word before the fp16 add, or MUL1's
//                (1024 + byte sum, 0);
//   B (32 x 16): the rotated input rows as duplicated pairs (x, x), activation row = B column;
//   D (16 x 16): 16 output columns x 16 activation rows, fp32.
// So the dot product of a decoded weight against every row costs the same matrix-core issue,
// whatever m is: the work per weight is the decode, as at m = 1.
//
// Lane mapping.  A unit of work is 2 column tiles x 4 k-tiles (8 tiles, 256 K bytes).  Lane l
// decodes tile (k-tile 4u + l / 16, column tile l % 16 / 8) of the wave's column pair as the
// M = 1 kernels do (lane j = l % 8 of its tile: columns j, j + 8, all 16 rows).  MFMA operand
// A's lane l must hold output column l % 16 and k-block l / 16: exactly this lane's column j
// (or j + 8) of its own k-tile.  The 8 MFMAs of a unit are (row group gq, column half c):
// A = the lane's decoded words 8 gq + 4 c .. + 3 (rows 2 gq, 2 gq + 1, 2 gq + 8, 2 gq + 9 of
// column j + 8 c), B = the input at those rows of the lane's k-tile, read as one 16-byte LDS
// load from the input staged in that row order (xperm).
//
// Workgroup: one 128-column chunk (4 waves = 4 column pairs) over SB k-tiles (SB % 8 == 0, so
// the input rotation covers whole 128-row chunks); split-k partials and their hand-off are the
// LDS kernel's (block_epilogue).
// ---------------------------------------------------------------------------------------------
typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));

// position of row rho (0..15) of a 16-row group in the staged input
__device__ __forceinline__ constexpr int xperm(int rho) { return 4 * ((rho & 7) >> 1) + (rho & 1) + 2 * (rho >> 3); }

template <int K, int CB, int MT>
__global__ __launch_bounds__(GEMV_THREADS)
void gemvm_kernel(const GemvArgs g)
{
    extern __shared__ __align__(16) uint32_t smem[];
    __shared__ int flag;
    __shared__ float sumx[MT];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t a3 = sconst(89226354u), b3 = vconst(64248484u);       // 3INST multiplier, addend
    const int m = g.m, k = g.k;
    const int KS = k / 16;
    const int SB = g.slices_per_block;                    // k-tiles per workgroup, multiple of 8
    const int splits = KS / SB;
    const int j = blockIdx.y;
    int chunk, slot;
    block_coords(g, splits, chunk, slot);
    MatView v;
    if (!resolve(g, j, v)) { inactive_arrive(g, chunk, slot, &flag); return; }
    if (chunk * 128 >= v.n) return;
    // the wave's start (staging) and end (hand-off) outrank the decode loops of the SIMD's other
    // waves, as in the M = 1 kernel
    __builtin_amdgcn_s_setprio(EXL3_GEMV_PRIO);
#ifdef EXL3_GEMV_TRACE
    {
        uint32_t hw, xcc;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)\n\ts_getreg_b32 %1, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(hw), "=s"(xcc));
        GEMV_STAMP(g, 0, hw);
        if (g.trace && (threadIdx.x & 63) == 0)
            g.trace[(((size_t) blockIdx.y * gridDim.x + blockIdx.x) * 4 + (threadIdx.x >> 6)) * 8 + 5] = ((uint64_t) xcc << 32) | hw;
    }
#endif
    const int ks0 = slot * SB;
    const int xs_stride = SB * 16 + 4;                    // u32 per row; +4: rows 16 bytes apart in the banks
    uint32_t* xs = smem;                                  // [MT][xs_stride] dup pairs, xperm order
    constexpr int RS = 132;                               // res row stride: 16-byte column groups of 16 rows in distinct banks
    float* res = (float*) (smem + MT * xs_stride);        // [MT][RS]
    float* tmp = res + MT * RS;                           // epilogue scratch: 2 x (m x 64 column pairs), >= 512

    // Input rotation of the workgroup's SB / 8 chunks, every row, into xs (dup pairs, xperm order).
    // Job q of wave w: row / chunk (w + 4 q) of m x SB / 8.  The first XB jobs' input and suh loads
    // are issued before the weight ring's: loads return in issue order, so behind the ring they
    // would wait for its HBM traffic.
    constexpr int XB = 4;                                 // measured best of 2 / 4 / 8 / 16 (m = 2..8)
    const int nkc = SB / 8, njobs = m * nkc;
    uint32_t xr[XB], sr[XB];
    auto xload = [&](int jb) {
        #pragma unroll
        for (int q = 0; q < XB; ++q)
        {
            const int job = min(jb + q * GEMV_WAVES, njobs - 1);
            const int row = job / nkc, c = job % nkc;
            const int col = ks0 * 16 + c * 128 + 2 * lane;
            xr[q] = *to_global((const uint32_t*) (v.A + (size_t) row * k + col));
            sr[q] = *to_global((const uint32_t*) ((v.suh ? v.suh : v.A) + col));   // unused without suh
        }
    };
    auto xstage = [&](int jb) {
        #pragma unroll
        for (int q = 0; q < XB; ++q)
        {
            const int job = jb + q * GEMV_WAVES;
            if (job >= njobs) break;
            const int row = job / nkc, c = job % nkc;
            f16x2 o = as_h2(xr[q]);
            if (v.suh)
            {
                const f16x2 xv = o * as_h2(sr[q]);
                float v0 = (float) xv.x, v1 = (float) xv.y;
                fwht128_wave(v0, v1, lane);
                o.x = (f16) (v0 * EXL3_HAD_RSCALE);
                o.y = (f16) (v1 * EXL3_HAD_RSCALE);
            }
            const int e = 2 * lane;                       // even row of its 16-group: xperm(e+1) = xperm(e) + 1
            const int pos = c * 128 + (e & ~15) + xperm(e & 15);
            f16x2 d0 = { o.x, o.x }, d1 = { o.y, o.y };
            *(u32x2*) (xs + row * xs_stride + pos) = (u32x2) { as_u32(d0), as_u32(d1) };
        }
    };
    xload(wave);
    __builtin_amdgcn_sched_barrier(0);

    // this lane's tile: k-tile ks0 + lane / 16 (+ 4 per unit), column tile 2 wave + lane % 16 / 8
    const int tiles_n = v.stride / 16;
    constexpr int KB = kbits(K);
    const int jt = lane & 7;
    const uint32_t* tile0 = (const uint32_t*) v.trellis
                          + ((size_t) (ks0 + (lane >> 4)) * tiles_n + chunk * 8 + 2 * wave + ((lane >> 3) & 1)) * tile_words(K);
    const size_t ustride = (size_t) 4 * tiles_n * tile_words(K);
    const int nunits = SB / 4;
    const int prev_off = jt == 0 ? 8 * K - 1 : -1;
    constexpr int PF = EXL3_GEMV_PF;
    uint32_t ring[PF][KB + 1];
    #pragma unroll
    for (int d = 0; d < PF; ++d) load_tile_lane<K>(tile0 + (size_t) min(d, nunits - 1) * ustride, jt, prev_off, ring[d]);
    // svh pair for the epilogue, behind the first weights
    const uint32_t svp = *to_global((const uint32_t*) ((v.svh ? v.svh + chunk * 128 : v.A) + 2 * lane));

    xstage(wave);
    for (int jb = wave + GEMV_WAVES * XB; jb < njobs; jb += GEMV_WAVES * XB)
    {
        xload(jb);
        xstage(jb);
    }
    __syncthreads();
    GEMV_STAMP(g, 1, 0);
    __builtin_amdgcn_s_setprio(0);

    const int nrow = min(lane & 15, m - 1);               // B column = activation row (clamped)
    const uint32_t* xb = xs + nrow * xs_stride + (lane >> 4) * 16;
    f32x4 acc[2] = { { 0, 0, 0, 0 }, { 0, 0, 0, 0 } };
    for (int u0 = 0; u0 < nunits; u0 += PF)
    {
        #pragma unroll
        for (int d = 0; d < PF; ++d)
        {
            const int u = u0 + d;
            if (u >= nunits) break;
            uint32_t wv[KB + 1];
            #pragma unroll
            for (int w = 0; w <= KB; ++w) wv[w] = ring[d][w];
            uint32_t raw[32];
            raw32<K, CB>(wv, raw, a3, b3);
            load_tile_lane<K>(tile0 + (size_t) min(u + PF, nunits - 1) * ustride, jt, prev_off, ring[d]);
            #pragma unroll
            for (int gq = 0; gq < 4; ++gq)
            {
                const u32x4 bx = *(const u32x4*) (xb + u * 64 + 4 * gq);
                const f16x8v b = __builtin_bit_cast(f16x8v, bx);
                #pragma unroll
                for (int c = 0; c < 2; ++c)
                {
                    const u32x4 aw = { raw[8 * gq + 4 * c], raw[8 * gq + 4 * c + 1], raw[8 * gq + 4 * c + 2], raw[8 * gq + 4 * c + 3] };
                    acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8v, aw), b, acc[c], 0, 0, 0);
                }
            }
        }
    }
    __builtin_amdgcn_s_setprio(EXL3_GEMV_PRIO);
    GEMV_STAMP(g, 2, __builtin_amdgcn_readfirstlane(__float_as_uint(acc[0].x + acc[1].x)));
    // D[i][n]: lane holds output columns i = 4 (lane / 16) + e of the wave's half c, row n = lane % 16
    const int n = lane & 15;
    if (n < m)
    {
        // the lane's 4 values are columns 32 wave + 16 (q >> 1) + 4 (q & 1) + 8 c + 0..3, q = lane / 16
        const int q = lane >> 4;
        #pragma unroll
        for (int c = 0; c < 2; ++c)
            *(f32x4*) (res + n * RS + 32 * wave + 16 * (q >> 1) + 4 * (q & 1) + 8 * c) = acc[c];
    }
    if (CB == 2)
    {
        // MUL1 bias term: sum of the rotated input over this workgroup's k range, per row
        for (int r = wave; r < m; r += GEMV_WAVES)
        {
            float sv = 0.0f;
            for (int e = lane; e < SB * 16; e += 64) sv += (float) as_h2(xs[r * xs_stride + e]).x;
            sv = wave_sum(sv, lane);
            if (lane == 0) sumx[r] = sv;
        }
    }
    __syncthreads();
    if (CB == 2)
    {
        const float kinv = (float) as_h(0x1eee);
        for (int e = threadIdx.x; e < m * 128; e += GEMV_THREADS)
        {
            float& rv = res[(e >> 7) * RS + (e & 127)];
            rv = rv * kinv + sumx[e >> 7] * (float) as_h(0xc931);
        }
        __syncthreads();
    }
    block_epilogue(g, v, j, chunk, slot, splits, res, tmp, &flag, svp, RS);
    GEMV_STAMP(g, 3, flag);
}

template <typename KernelLaunch>
int launch_common(const GemvArgs& g, hipStream_t s, KernelLaunch main)
{
    const int KS = g.k / 16;
    const int splits = KS / g.slices_per_block;
    const int chunks = g.n / 128;
    main(dim3(splits * chunks, g.bszm));
    if (!g.xcd)
    {
        if (splits > 1)
            hipLaunchKernelGGL(gemv_finish, dim3(chunks, g.bszm), dim3(GEMV_THREADS), 0, s, g, splits);
        if (g.weights)
            hipLaunchKernelGGL(gemv_weighted_reduce, dim3(chunks), dim3(GEMV_THREADS), 0, s, g);
    }
    return (int) hipGetLastError();
}

template <int K, int CB, int MT>
int launch_gemv_t(const GemvArgs& g, hipStream_t s)
{
    const size_t lds = (size_t) MT * g.xs_chunks * 128 * 4 + (size_t) GEMV_WAVES * MT * 128 * 4;
    return launch_common(g, s, [&](dim3 grid) {
        hipLaunchKernelGGL((gemv_kernel<K, CB, MT>), grid, dim3(GEMV_THREADS), lds, s, g);
    });
}

template <int K, int CB, int IN>
void launch_gemv1_in(const GemvArgs& g, hipStream_t s, dim3 grid)
{
    const int W = g.slices_per_block / GEMV_WAVES;
    if (W == 1) hipLaunchKernelGGL((gemv1_kernel<K, CB, 1, IN>), grid, dim3(GEMV_THREADS), 0, s, g);
    else if (W == 2) hipLaunchKernelGGL((gemv1_kernel<K, CB, 2, IN>), grid, dim3(GEMV_THREADS), 0, s, g);
    else if (W == 4) hipLaunchKernelGGL((gemv1_kernel<K, CB, 4, IN>), grid, dim3(GEMV_THREADS), 0, s, g);
    else hipLaunchKernelGGL((gemv1_kernel<K, CB, 8, IN>), grid, dim3(GEMV_THREADS), 0, s, g);
}

template <int K, int CB>
int launch_gemv1(const GemvArgs& g, hipStream_t s)
{
    return launch_common(g, s, [&](dim3 grid) {
        if (g.A_up) launch_gemv1_in<K, CB, GEMV_IN_SILU>(g, s, grid);
        else if (g.in_w) launch_gemv1_in<K, CB, GEMV_IN_NORM>(g, s, grid);
        else launch_gemv1_in<K, CB, GEMV_IN_PLAIN>(g, s, grid);
    });
}

template <int K, int CB, int MT>
int launch_gemvm_t(const GemvArgs& g, hipStream_t s)
{
    const size_t lds = ((size_t) MT * (g.slices_per_block * 16 + 4) + (size_t) MT * 132 + (MT * 128 > 512 ? MT * 128 : 512)) * 4;
    return launch_common(g, s, [&](dim3 grid) {
        hipLaunchKernelGGL((gemvm_kernel<K, CB, MT>), grid, dim3(GEMV_THREADS), lds, s, g);
    });
}

template <int K, int CB>
int launch_gemv_m(const GemvArgs& g, hipStream_t s)
{
    if (g.m == 1 && g.stream_m1 == 2)
    {
        if constexpr (CB == 2) return -1;                // (the planner never picks it for MUL1)
        else
        {
            const int waves = g.bszm * (g.n / 128) * (g.k / 16) / g.slices_per_block;
            hipLaunchKernelGGL((gemv1b_kernel<K, CB>), dim3(waves / GEMV_WAVES), dim3(GEMV_THREADS), 0, s, g);
            return (int) hipGetLastError();
        }
    }
    if (g.m == 1 && g.stream_m1) return launch_gemv1<K, CB>(g, s);
    if (g.A_up || g.in_w) return -1;   // the fused input forms exist in the M = 1 stream kernel only
    if (g.mfma_rows)
    {
        if (g.m == 1) return launch_gemvm_t<K, CB, 1>(g, s);
        if (g.m <= 4) return launch_gemvm_t<K, CB, 4>(g, s);
        if (g.m <= 8) return launch_gemvm_t<K, CB, 8>(g, s);
        return launch_gemvm_t<K, CB, 16>(g, s);
    }
    if (g.m == 1) return launch_gemv_t<K, CB, 1>(g, s);
    if (g.m <= 4) return launch_gemv_t<K, CB, 4>(g, s);
    return launch_gemv_t<K, CB, 8>(g, s);
}

}  // namespace

#define EXL3_CAT2(a, b) a##b
#define EXL3_CAT(a, b) EXL3_CAT2(a, b)

int EXL3_CAT(exl3k_gemv_k, EXL3_INST_K)(const GemvArgs& g, int cb, hipStream_t s)
{
#if EXL3_INST_K >= 16
    return cb == 2 ? launch_gemv_m<EXL3_INST_K, 2>(g, s) : -1;     // half rates: mul1 only
#else
    switch (cb)
    {
        case 0: return launch_gemv_m<EXL3_INST_K, 0>(g, s);
        case 1: return launch_gemv_m<EXL3_INST_K, 1>(g, s);
        case 2: return launch_gemv_m<EXL3_INST_K, 2>(g, s);
    }
    return -1;
#endif
}
