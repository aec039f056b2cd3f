// Issue-rate microbenchmarks for gfx950 (libexl3_probe.so, driven by `bench.py --rates`).
//
// The decode-cost arguments of the EXL3 kernels rest on these rates: how many wave64 VALU
// instructions of each kind a SIMD issues per clock, and how fast the LDS serves random 16-bit
// gathers from a 128 KiB table (the alternative to decoding a codebook in registers).
//
// Each VALU probe runs NCH independent chains per lane (no dependency stalls), ITER iterations of
// UNR instructions each, over a grid of W waves per SIMD on every CU; one lane per wave stores a
// checksum with a vector store so that nothing is dead code.  The host times the launch with HIP
// events and reports instructions per SIMD per nanosecond; the ratio to the base-rate probe
// (v_add_u32 is dual-issue on gfx950, so v_bfe_u32 is the base) is clock-independent.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int NCH = 8;       // independent chains per lane
constexpr int UNR = 16;      // instructions per chain per iteration (unrolled)

enum Op
{
    OP_BFE = 0,         // v_bfe_u32
    OP_MAD64 = 1,       // v_mad_u64_u32 (low word used)
    OP_BITOP3 = 2,      // v_bitop3_b32
    OP_MAD_U32_U16 = 3, // v_mad_u32_u16
    OP_PERM = 4,        // v_perm_b32
    OP_ALIGNBIT = 5,    // v_alignbit_b32
    OP_DOT2 = 6,        // v_dot2_f32_f16
    OP_PK_FMA_F16 = 7,  // v_pk_fma_f16
    OP_ADD = 8,         // v_add_u32
    OP_MUL_LO = 9,      // v_mul_lo_u32
    OP_COUNT = 10,
};

template <int OP>
__device__ __forceinline__ void step(uint32_t& v, uint32_t a, uint32_t b)
{
    if constexpr (OP == OP_BFE) asm volatile("v_bfe_u32 %0, %0, %1, 16" : "+v"(v) : "s"(a));
    else if constexpr (OP == OP_MAD64)
    {
        uint64_t r;
        asm volatile("v_mad_u64_u32 %0, vcc, %1, %2, %3" : "=v"(r) : "v"(v), "s"(a), "v"((uint64_t) b) : "vcc");
        v = (uint32_t) r;
    }
    else if constexpr (OP == OP_BITOP3) asm volatile("v_bitop3_b32 %0, %0, %1, %2 bitop3:0x6a" : "+v"(v) : "s"(a), "v"(b));
    else if constexpr (OP == OP_MAD_U32_U16) asm volatile("v_mad_u32_u16 %0, %0, %1, %2" : "+v"(v) : "s"(a), "v"(b));
    else if constexpr (OP == OP_PERM) asm volatile("v_perm_b32 %0, %0, %2, %1" : "+v"(v) : "s"(a), "v"(b));
    else if constexpr (OP == OP_ALIGNBIT) asm volatile("v_alignbit_b32 %0, %0, %1, 7" : "+v"(v) : "v"(b));
    else if constexpr (OP == OP_DOT2)
    {
        float f = __builtin_bit_cast(float, v);
        asm volatile("v_dot2_f32_f16 %0, %1, %2, %0" : "+v"(f) : "v"(b), "s"(a));
        v = __builtin_bit_cast(uint32_t, f);
    }
    else if constexpr (OP == OP_PK_FMA_F16) asm volatile("v_pk_fma_f16 %0, %0, %1, %2" : "+v"(v) : "s"(a), "v"(b));
    else if constexpr (OP == OP_ADD) asm volatile("v_add_u32 %0, %0, %1" : "+v"(v) : "v"(b));
    else if constexpr (OP == OP_MUL_LO) asm volatile("v_mul_lo_u32 %0, %0, %1" : "+v"(v) : "s"(a));
}

template <int OP>
__global__ __launch_bounds__(256) void valu_probe(uint32_t* out, int iters, uint32_t a, uint32_t b0)
{
    uint32_t v[NCH];
    const uint32_t b = b0 ^ threadIdx.x;
    #pragma unroll
    for (int c = 0; c < NCH; ++c) v[c] = threadIdx.x * 2654435761u + c;
    for (int it = 0; it < iters; ++it)
    {
        #pragma unroll
        for (int u = 0; u < UNR; ++u)
        {
            #pragma unroll
            for (int c = 0; c < NCH; ++c) step<OP>(v[c], a, b);
        }
    }
    uint32_t s = 0;
    #pragma unroll
    for (int c = 0; c < NCH; ++c) s ^= v[c];
    if ((threadIdx.x & 63) == 0) out[blockIdx.x * 4 + (threadIdx.x >> 6)] = s;
}

// Random 16-bit gathers from a 128 KiB LDS table: 1024 threads per workgroup (one workgroup per
// CU, 4 waves per SIMD), NCH chains per lane.  The next byte address of a chain is
// (x * 47 + value) & 0x1fffe: one v_mad_u32_u24 and one v_and_b32 per gather.  `mode` 1 runs the
// same VALU without the LDS reads (the VALU share of the loop).
__global__ __launch_bounds__(1024) void lds_gather_probe(uint32_t* out, int iters, int mode)
{
    extern __shared__ __align__(16) uint16_t table[];    // 65536 entries
    for (int i = threadIdx.x; i < 65536; i += 1024) table[i] = (uint16_t) (i * 40503u);
    __syncthreads();
    uint32_t x[NCH];
    #pragma unroll
    for (int c = 0; c < NCH; ++c) x[c] = (threadIdx.x * 2654435761u + c * 40503u) & 0x1fffeu;
    for (int it = 0; it < iters; ++it)
    {
        #pragma unroll
        for (int u = 0; u < UNR; ++u)
        {
            #pragma unroll
            for (int c = 0; c < NCH; ++c)
            {
                const uint32_t r = mode == 0 ? (uint32_t) *(const uint16_t*) ((const char*) table + x[c]) : x[c] >> 3;
                x[c] = (__umul24(x[c], 47u) + r) & 0x1fffeu;
            }
        }
    }
    uint32_t acc = 0;
    #pragma unroll
    for (int c = 0; c < NCH; ++c) acc ^= x[c];
    if ((threadIdx.x & 63) == 0) out[blockIdx.x * 16 + (threadIdx.x >> 6)] = acc;
}

// Read-only streaming probe: `bytes` (a multiple of 1 KiB * wgs * 4) read with 16-byte loads,
// 4 waves per workgroup, one 1 KiB block per wave per step, 2 blocks in flight per wave (the
// GEMV's ring depth); one lane per wave stores an xor checksum.
//   pattern 0: the blocks of a wave are contiguous (wave w reads bytes [w B, (w + 1) B));
//   pattern 1: the GEMV's order: the matrix is `rows` rows of `row_bytes`, wave w reads the 1 KiB
//              column block w % (row_bytes / 1 KiB) of rows (w / cols) * R .. + R (stride row_bytes).
typedef uint32_t pu32x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void stream_probe(const pu32x4* __restrict__ buf, size_t blocks_per_wave, int pattern,
                                                    size_t row_blocks, uint32_t* out)
{
    const int lane = threadIdx.x & 63;
    const size_t w = (size_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    size_t b0, stride;
    if (pattern == 0) { b0 = w * blocks_per_wave; stride = 1; }
    else
    {
        const size_t col = w % row_blocks, grp = w / row_blocks;
        b0 = grp * blocks_per_wave * row_blocks + col;
        stride = row_blocks;
    }
    pu32x4 acc = { 0u, 0u, 0u, 0u };
    pu32x4 r0 = __builtin_nontemporal_load(buf + b0 * 64 + lane);
    pu32x4 r1 = __builtin_nontemporal_load(buf + (b0 + (blocks_per_wave > 1 ? stride : 0)) * 64 + lane);
    for (size_t i = 2; i < blocks_per_wave + 2; i += 2)
    {
        const size_t i0 = i < blocks_per_wave ? i : blocks_per_wave - 1, i1 = i + 1 < blocks_per_wave ? i + 1 : blocks_per_wave - 1;
        acc.x ^= r0.x; acc.y ^= r0.y; acc.z ^= r0.z; acc.w ^= r0.w;
        r0 = __builtin_nontemporal_load(buf + (b0 + i0 * stride) * 64 + lane);
        acc.x ^= r1.x; acc.y ^= r1.y; acc.z ^= r1.z; acc.w ^= r1.w;
        r1 = __builtin_nontemporal_load(buf + (b0 + i1 * stride) * 64 + lane);
    }
    const uint32_t v = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (lane == 0) out[w] = v;
}

template <int OP>
hipError_t launch_valu(uint32_t* out, int blocks, int iters, hipStream_t s)
{
    hipLaunchKernelGGL((valu_probe<OP>), dim3(blocks), dim3(256), 0, s, out, iters, 0x3b603b60u, 0x12345678u);
    return hipGetLastError();
}

}  // namespace

extern "C" {

int exl3_probe_valu_ops(void) { return OP_COUNT; }
int exl3_probe_chains(void) { return NCH * UNR; }

// Time one VALU probe: blocks workgroups of 4 waves, iters iterations of NCH * UNR instructions
// per lane.  Returns milliseconds (< 0: HIP error).  out: 4 * blocks uint32.
float exl3_probe_valu(int op, uint32_t* out, int blocks, int iters)
{
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1.0f;
    (void) hipEventRecord(e0, nullptr);
    hipError_t rc = hipErrorInvalidValue;
    switch (op)
    {
        case OP_BFE: rc = launch_valu<OP_BFE>(out, blocks, iters, nullptr); break;
        case OP_MAD64: rc = launch_valu<OP_MAD64>(out, blocks, iters, nullptr); break;
        case OP_BITOP3: rc = launch_valu<OP_BITOP3>(out, blocks, iters, nullptr); break;
        case OP_MAD_U32_U16: rc = launch_valu<OP_MAD_U32_U16>(out, blocks, iters, nullptr); break;
        case OP_PERM: rc = launch_valu<OP_PERM>(out, blocks, iters, nullptr); break;
        case OP_ALIGNBIT: rc = launch_valu<OP_ALIGNBIT>(out, blocks, iters, nullptr); break;
        case OP_DOT2: rc = launch_valu<OP_DOT2>(out, blocks, iters, nullptr); break;
        case OP_PK_FMA_F16: rc = launch_valu<OP_PK_FMA_F16>(out, blocks, iters, nullptr); break;
        case OP_ADD: rc = launch_valu<OP_ADD>(out, blocks, iters, nullptr); break;
        case OP_MUL_LO: rc = launch_valu<OP_MUL_LO>(out, blocks, iters, nullptr); break;
    }
    (void) hipEventRecord(e1, nullptr);
    float ms = -1.0f;
    if (rc == hipSuccess && hipEventSynchronize(e1) == hipSuccess) (void) hipEventElapsedTime(&ms, e0, e1);
    (void) hipEventDestroy(e0);
    (void) hipEventDestroy(e1);
    return rc == hipSuccess ? ms : -1.0f;
}

// Time the LDS gather probe (mode 0) or its VALU-only twin (mode 1).  out: 16 * blocks uint32.
float exl3_probe_lds_gather(uint32_t* out, int blocks, int iters, int mode)
{
    if (hipFuncSetAttribute((const void*) lds_gather_probe, hipFuncAttributeMaxDynamicSharedMemorySize, 131072) !=
        hipSuccess)
        return -1.0f;
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1.0f;
    (void) hipEventRecord(e0, nullptr);
    hipLaunchKernelGGL(lds_gather_probe, dim3(blocks), dim3(1024), 131072, nullptr, out, iters, mode);
    const hipError_t rc = hipGetLastError();
    (void) hipEventRecord(e1, nullptr);
    float ms = -1.0f;
    if (rc == hipSuccess && hipEventSynchronize(e1) == hipSuccess) (void) hipEventElapsedTime(&ms, e0, e1);
    (void) hipEventDestroy(e0);
    (void) hipEventDestroy(e1);
    return rc == hipSuccess ? ms : -1.0f;
}

// One streaming launch on `stream` (no timing: the caller times a sequence, e.g. in a graph).
// bytes must be a multiple of 1 KiB * 4 * wgs; pattern 1 also needs row_bytes % 1 KiB == 0 and
// (bytes / row_bytes) % (waves / (row_bytes / 1 KiB)) == 0.  Returns 0 or a HIP error.
int exl3_probe_stream(const void* buf, size_t bytes, int wgs, int pattern, size_t row_bytes, uint32_t* out, void* stream)
{
    const size_t waves = (size_t) wgs * 4, blocks = bytes / 1024;
    if (!buf || !out || wgs <= 0 || blocks % waves) return (int) hipErrorInvalidValue;
    size_t row_blocks = 1;
    if (pattern == 1)
    {
        row_blocks = row_bytes / 1024;
        const size_t rows = bytes / row_bytes;
        if (row_bytes % 1024 || bytes % row_bytes || waves % row_blocks || rows % (waves / row_blocks)) return (int) hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(stream_probe, dim3(wgs), dim3(256), 0, (hipStream_t) stream, (const pu32x4*) buf, blocks / waves,
                       pattern, row_blocks, out);
    return (int) hipGetLastError();
}

}  // extern "C"
