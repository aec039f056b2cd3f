// Internal launcher interface between the C-ABI layer (exl3_capi.cpp) and the kernel units.
// Launchers validate nothing: the C-ABI checks every shape, pointer and bitrate first.
// They return 0 or a hipError_t / -1 (no instance for the requested K / codebook).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

struct GemvArgs
{
    const uint16_t* A;          // (m, k) fp16
    const uint16_t* trellis;    // (k/16, n/16, 16K) uint16
    void* C;                    // (m, n) fp16 or fp32
    const uint16_t* suh;        // (k) fp16 or null
    const uint16_t* svh;        // (n) fp16 or null
    int m, k, n;
    int c_fp32;
    int stream_m1;              // 1: M = 1 streaming kernel (SB % 32 == 0), 0: LDS kernel
    int slices_per_block;       // SB: k-slices (16 rows x 128 columns) per workgroup, divides k/16
    int slots;                  // split partials per column chunk: k/16 / SB
    int xs_chunks;              // rotated 128-row input chunks held in LDS: SB/8 + 2
    int xcd;                    // > 0: XCD-local split-k hand-off over this many XCDs (M = 1 stream)
    float* partials;            // workspace: slots * m * n fp32
    int* counters;              // workspace: n / 128 ints (kernels that hand off through counters)
};

int exl3k_reconstruct(uint16_t* W, const uint16_t* trellis, int k, int n, int tiles_n,
                      int nt_off, int K, int cb, hipStream_t s);
int exl3k_reconstruct_had(uint16_t* W, const uint16_t* trellis, const uint16_t* suh,
                          const uint16_t* svh, int k, int n, int tiles_n, int nt_off,
                          int K, int cb, hipStream_t s);

int exl3k_xcd_probe(int* out, int blocks, hipStream_t s);

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
