// Internal launcher interface between the C-ABI layer (exl3_capi.cpp) and the kernel units.
// Launchers validate nothing: the C-ABI checks every shape, pointer and bitrate first.
// They return 0 or a hipError_t / -1 (no instance for the requested K / codebook).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// One GEMV launch over bszm "slots" (grid.y).  Single-matrix exl3_gemm: bszm = 1 and the
// direct pointers.  Multi-matrix exl3_mgemm: device pointer tables, resolved per slot in the
// kernel (quant/exl3_gemm_kernel.cuh:88-343 semantics).
struct GemvArgs
{
    const uint16_t* A;          // (bszm_in, m, k) fp16
    const uint16_t* trellis;    // (k/16, n/16, 16K) uint16 (single matrix)
    void* C;                    // (bszm, m, n) fp16 or fp32
    const uint16_t* suh;        // (k) fp16 or null (single matrix)
    const uint16_t* svh;        // (n) fp16 or null (single matrix)
    int m, k, n;                // n: output width (the maximum width with size_n)
    int c_fp32;
    // multi-matrix tables (all device memory; null when unused)
    const uint64_t* B_list;     // trellis pointer per matrix (non-null selects table mode)
    const uint64_t* suh_list;   // suh pointer per matrix, or per source in sliced mode
    const uint64_t* svh_list;   // svh pointer per matrix
    const int64_t* indices;     // slot -> matrix, negative = inactive slot
    const uint16_t* weights;    // fp16 routing weight per slot: outputs summed per token group
    const int* size_n;          // per-matrix output width
    const uint64_t* c_list;     // per-matrix output pointer
    const int* n_stride;        // per-matrix row stride of trellis tiles and C (sliced mode)
    const int* had_src;         // per-matrix input source (sliced mode)
    int bszm_in;                // input slabs: 1 = broadcast
    int bszm;                   // slots (grid.y)
    int num_tokens;             // weighted reduction groups
    // work split (host planner)
    int stream_m1;              // 1: M = 1 streaming kernel, 0: LDS kernel
    int slices_per_block;       // SB: k-slices (16 rows x 128 columns) per workgroup, divides k/16
    int slots;                  // split partials per column chunk: k/16 / SB
    int xs_chunks;              // rotated 128-row input chunks held in LDS (LDS kernel)
    int xcd;                    // > 0: XCD-local hand-off through L2 counters (workgroup b on XCD b % xcd)
    float* partials;            // workspace: bszm * slots * m * n fp32
    int* counters;              // workspace: zeroed; [0, half) per (slot, chunk), [half, ..) per chunk
    int counters_half;
    uint64_t* trace;            // instrumented builds only (EXL3_GEMV_TRACE): per-wave timestamps
};

// Prefill GEMM (m > 8) over the rotated input.
struct GemmArgs
{
    const uint16_t* A_rot;      // (m, k) fp16: had(A o suh) (the caller's A_had) or A itself
    const uint16_t* trellis;    // (k/16, n/16, 16K) uint16
    void* C;                    // (m, n) fp16 or fp32
    const uint16_t* svh;        // (n) fp16 or null
    int m, k, n;
    int c_fp32;
};

int exl3k_gemm_k1(const GemmArgs& g, int cb, hipStream_t s);
int exl3k_gemm_k2(const GemmArgs& g, int cb, hipStream_t s);
int exl3k_gemm_k3(const GemmArgs& g, int cb, hipStream_t s);
int exl3k_gemm_k4(const GemmArgs& g, int cb, hipStream_t s);
int exl3k_gemm_k5(const GemmArgs& g, int cb, hipStream_t s);
int exl3k_gemm_k6(const GemmArgs& g, int cb, hipStream_t s);
int exl3k_gemm_k7(const GemmArgs& g, int cb, hipStream_t s);
int exl3k_gemm_k8(const GemmArgs& g, int cb, hipStream_t s);

int exl3k_reconstruct(uint16_t* W, const uint16_t* trellis, int k, int n, int tiles_n,
                      int nt_off, int K, int cb, hipStream_t s);
int exl3k_reconstruct_had(uint16_t* W, const uint16_t* trellis, const uint16_t* suh,
                          const uint16_t* svh, int k, int n, int tiles_n, int nt_off,
                          int K, int cb, hipStream_t s);

int exl3k_xcd_probe(int* out, int blocks_x, int blocks_y, hipStream_t s);
int exl3k_mgemm_filter(const int64_t* indices, const uint16_t* weights, int bszm, int min_index,
                       int max_index, int num_tokens, int64_t* idx_out, uint16_t* w_out, hipStream_t s);

int exl3k_had128(const void* in, void* out, int rows, int cols, int fp32,
                 const uint16_t* pre, const uint16_t* post, float scale, hipStream_t s);

int exl3k_gemv_k1(const GemvArgs& g, int cb, hipStream_t s);
int exl3k_gemv_k2(const GemvArgs& g, int cb, hipStream_t s);
int exl3k_gemv_k3(const GemvArgs& g, int cb, hipStream_t s);
int exl3k_gemv_k4(const GemvArgs& g, int cb, hipStream_t s);
int exl3k_gemv_k5(const GemvArgs& g, int cb, hipStream_t s);
int exl3k_gemv_k6(const GemvArgs& g, int cb, hipStream_t s);
int exl3k_gemv_k7(const GemvArgs& g, int cb, hipStream_t s);
int exl3k_gemv_k8(const GemvArgs& g, int cb, hipStream_t s);
