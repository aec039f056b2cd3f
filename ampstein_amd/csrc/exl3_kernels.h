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
    int slab_m;                 // rows per A / C slab (0: m); a launch may cover rows [row0, row0 + m)
    int row0;
    // work split (host planner)
    int stream_m1;              // 2: M = 1 balanced stream, 1: M = 1 streaming kernel, 0: LDS kernel
    int p1_blocks;              // balanced stream: workgroups (a multiple of xcd)
    int slices_per_block;       // SB: k-slices (16 rows x 128 columns) per workgroup, divides k/16
    int slots;                  // split partials per column chunk: k/16 / SB
    int xs_chunks;              // rotated 128-row input chunks held in LDS (LDS kernel)
    int xcd;                    // > 0: XCD-local hand-off through L2 counters (workgroups b and b + xcd on one XCD)
    const uint32_t* sink;       // workspace: 8 KiB never written, target of the stream's past-the-end prefetches
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

// Fused decode-shaped MoE (exl3_moe_coop): route/rotate, gate/up GEMV + activation, down GEMV +
// routing-weighted sum.  Device pointers throughout; tables indexed by local expert.
struct MoeArgs
{
    const uint16_t* x;          // (bsz, H) fp16, row stride x_stride
    int x_stride;
    const int64_t* sel;         // (bsz, topk) expert indices
    const uint16_t* rw;         // (bsz, topk) fp16 routing weights (0 = inactive slot)
    int bsz, topk, H, Hi, I, Ho, H_out;
    int min_expert, max_expert; // min < 0: no range filter
    const uint64_t *g_trellis, *g_suh, *g_svh;
    const uint64_t *u_trellis, *u_suh, *u_svh;
    const uint64_t *d_trellis, *d_suh, *d_svh;
    const uint64_t *g_bias, *u_bias, *d_bias;      // nullable tables of fp16 vectors
    const uint8_t *g_bits, *u_bits, *d_bits;       // per-expert widths (mixed K), or null
    int K_gu, K_d;              // uniform widths when the tables are null
    int act;                    // 0 SiLU, 1 GELU (tanh), 2 ReLU^2, 3 clamped SwiGLU (gpt-oss)
    float act_limit;
    int gated;                  // 0: no gate projection, activation relu(u) * u
    uint16_t* had_g;            // (slots_max, Hi) rotated gate input
    uint16_t* had_u;            // (slots_max, Hi) rotated up input
    uint16_t* act_out;          // (slots_max, I) activation, rotated for the down projection
    int* runs;                  // run table in the caller's ctr: [n_runs, -, run_start[slots_max+1], order[slots_max]]
    int slots_max;
    float* out;                 // (bsz, H_out) fp32, row stride out_stride
    int out_stride;
    const float* sh_out;        // shared expert output (bsz, H) fp32, or null
    const uint16_t* sh_gate_w;  // (H) fp16 shared-expert gate weight, or null
    // library workspace
    float* part_a;              // [2][splits_a][slots][I] gate/up partials
    float* part_b;              // [splits_b][slots][Ho] down partials
    int* ctr_a;                 // [slots][I/128] x 32 (one 128-byte line each)
    int* ctr_b;                 // [bsz][Ho/128] x 32
    int splits_a, splits_b;
    int xcd;                    // > 0: chunk c runs on XCD c % xcd (workgroup-scope hand-off)
    int run_lo, run_hi;         // this launch takes the runs of run_lo + 1 .. run_hi slots
};

int exl3k_moe_cb0(const MoeArgs& a, hipStream_t s);
int exl3k_moe_cb1(const MoeArgs& a, hipStream_t s);
int exl3k_moe_cb2(const MoeArgs& a, hipStream_t s);
constexpr int EXL3_MOE_SBMAX = 64;     // k-slices per workgroup of the MoE GEMV (LDS bound)

int exl3k_reconstruct(uint16_t* W, const uint16_t* trellis, int k, int n, int tiles_n,
                      int nt_off, int K, int cb, hipStream_t s);
int exl3k_reconstruct_tr(uint16_t* WT, const uint16_t* trellis, int k, int n, int tiles_n,
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
int exl3k_gemv_k17(const GemvArgs& g, int cb, hipStream_t s);     // 1.5 bits (mul1)
int exl3k_gemv_k18(const GemvArgs& g, int cb, hipStream_t s);     // 2.5
int exl3k_gemv_k19(const GemvArgs& g, int cb, hipStream_t s);     // 3.5
