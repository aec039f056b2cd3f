// Internal launcher interface between the C-ABI layer (exl3_capi.cpp) and the kernel units.
// Launchers validate nothing: the C-ABI checks every shape, pointer and bitrate first.
// They return 0 or a hipError_t / -1 (no instance for the requested K / codebook).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// Per-launch check of the XCD-local hand-off.  The hand-off publishes split-k partials with a
// workgroup-scope release, which does not write the XCD's L2 back: the last arrival at a counter
// sees the other arrivals' partials only when they ran on its XCD.  The library enables it after
// the init probe has seen round-robin dispatch (workgroup b on XCD (b0 + b) % xcd); this guard
// checks the assumption at every counter, every launch: the counter is a 64-bit word that also
// sums the arrivals' XCC ids and their squares, and the last arrival stores 1 to the host-visible
// alarm word when the ids differ (exl3_xcd.cuh).  The host reads the alarm at every call and,
// once it is set, turns the hand-off off for the device (the finish kernel and agent-scope paths
// sum the partials instead).
struct XcdGuard
{
    uint32_t* alarm;            // pinned host word (device-mapped), 0 until a mixed arrival is seen
    int fake_block;             // test hook: linear workgroup that reports XCC id + 1 (-1: none)
};

// Workgroup -> hand-off coordinates of the GEMV kernels (grid.x = splits x chunks).  XCD mode: the
// splits of chunk c are workgroups b with b % xcd == c % xcd.  Shared with the host-side mapping
// check (exl3_amd_debug_handoff_map).
__host__ __device__ inline void gemv_block_coords(int xcd, int splits, int b, int& chunk, int& slot)
{
    if (xcd > 0)
    {
        const int xb = b % xcd, lb = b / xcd;
        chunk = xb + xcd * (lb / splits);
        slot = lb % splits;
    }
    else
    {
        chunk = b / splits;
        slot = b - chunk * splits;
    }
}

// MoE stages: workgroup b -> (column chunk, rest = split / projection / run).  XCD mode: chunk
// c's workgroups are b with b % xcd == c % xcd (chunks % xcd == 0).
__host__ __device__ inline void moe_chunk_coords(int xcd, int chunks, int b, int& chunk, int& rest)
{
    if (xcd > 0)
    {
        const int x = b % xcd, lb = b / xcd, cq = chunks / xcd;
        chunk = x + xcd * (lb % cq);
        rest = lb / cq;
    }
    else
    {
        chunk = b % chunks;
        rest = b / chunks;
    }
}

// Balanced M = 1 stream (gemv1b_kernel): the pairs p = j * chunks + chunk of residue x = b % xcd
// are concatenated, KS slices each; workgroup b (local index lb = b / xcd) streams slices
// [4 R lb, 4 R lb + 4 R) of that list, covering the tail of pair pa and the head of pair pb at most.
// Returns false for a workgroup past the list's end.  first / count: the local indices that
// contribute to the pair with list position q.
struct Gemv1bBlock { int pa, pb, qA; bool straddle; };
__host__ __device__ inline bool gemv1b_block(int xcd, int pairs, int KS, int R, int b, Gemv1bBlock& o)
{
    const int xq = b % xcd, lb = b / xcd;
    const int per_x = pairs / xcd;
    const int T0 = lb * 4 * R;
    if (T0 >= per_x * KS) return false;
    o.qA = T0 / KS;
    o.straddle = T0 + 4 * R > (o.qA + 1) * KS;
    o.pa = xq + xcd * o.qA;
    o.pb = o.straddle ? o.pa + xcd : o.pa;
    return true;
}
__host__ __device__ inline void gemv1b_pair_span(int KS, int R, int q, int& first, int& count)
{
    const int WR = 4 * R;
    first = (q * KS) / WR;
    count = ((q + 1) * KS - 1) / WR - first + 1;
}

// One GEMV launch over bszm "slots" (grid.y).  Single-matrix exl3_gemm: bszm = 1 and the
// direct pointers.  Multi-matrix exl3_mgemm: device pointer tables, resolved per slot in the
// kernel (quant/exl3_gemm_kernel.cuh:88-343 semantics).
struct GemvArgs
{
    const uint16_t* A;          // (bszm_in, m, k) fp16
    const uint16_t* A_up;       // non-null: the input is fp16(silu(A) * A_up) (M = 1 stream kernel only)
    // non-null norm_h: after the row is complete, norm_h = fp16(norm_h + C) and
    // norm_r = rmsnorm(norm_h) * norm_w (M = 1 stream kernel, single matrix, fp16 C, one split or XCD hand-off)
    uint16_t* norm_h;
    const uint16_t* norm_w;
    uint16_t* norm_r;
    int* norm_ctr;              // workspace counter on its own 128-byte line, zero between calls
    float norm_eps;
    // non-null res_h (producer of a split residual norm): after C is stored, res_h = fp16(res_h + C)
    // and res_sq[row * (n / 128) + chunk] = that chunk's fp32 sum of squares (single matrix, fp16 C)
    uint16_t* res_h;
    float* res_sq;
    // non-null in_w (consumer of a split residual norm; M = 1 stream kernel, k <= 32768): the
    // input is fp16(fp16(A * scale) * in_w), scale = 1 / sqrt(sum(in_sq[0 .. k/128)) / k + in_eps)
    const float* in_sq;
    const uint16_t* in_w;
    float in_eps;
    uint16_t* in_r;             // (m, k) scratch for the other kernels: the normalised input is formed there first
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
    int stream_m1;              // 1: M = 1 streaming kernel, 0: LDS kernel
    int mfma_rows;              // 1: row-batched matrix-core kernel (gemvm_kernel, m <= 16)
    int slices_per_block;       // SB: k-slices (16 rows x 128 columns) per workgroup, divides k/16
    int slots;                  // split partials per column chunk: k/16 / SB
    int xs_chunks;              // rotated 128-row input chunks held in LDS (LDS kernel)
    int xcd;                    // > 0: XCD-local hand-off through L2 counters (workgroups b and b + xcd on one XCD)
    const uint32_t* sink;       // workspace: 8 KiB never written, target of the stream's past-the-end prefetches
    float* partials;            // workspace: bszm * slots * m * n fp32
    int* counters;              // workspace: zeroed; [0, half) per (slot, chunk), [half, ..) per chunk;
                                // XCD mode: 64-bit at each 128-byte line
    int counters_half;
    XcdGuard xg;                // hand-off check (used when xcd > 0)
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
    int reg_staging;            // 1: register-staged operands (gemm_kernel) instead of LDS DMA
    int splits;                 // > 1 (LDS-DMA form): k split in that many ranges per 256 x 256 tile,
    float* part;                //   fp32 partial tiles here (splits x tiles x 256 KiB), then the fixup
};

int exl3k_gemm_k1(const GemmArgs& g, int cb, hipStream_t s);
int exl3k_gemm_k2(const GemmArgs& g, int cb, hipStream_t s);
int exl3k_gemm_k3(const GemmArgs& g, int cb, hipStream_t s);
int exl3k_gemm_k4(const GemmArgs& g, int cb, hipStream_t s);
int exl3k_gemm_k5(const GemmArgs& g, int cb, hipStream_t s);
int exl3k_gemm_k6(const GemmArgs& g, int cb, hipStream_t s);
int exl3k_gemm_k7(const GemmArgs& g, int cb, hipStream_t s);
int exl3k_gemm_k8(const GemmArgs& g, int cb, hipStream_t s);
int exl3k_gemm_k17(const GemmArgs& g, int cb, hipStream_t s);   // half rates 1.5 / 2.5 / 3.5: mul1
int exl3k_gemm_k18(const GemmArgs& g, int cb, hipStream_t s);
int exl3k_gemm_k19(const GemmArgs& g, int cb, hipStream_t s);

// Grouped GEMM of the token-sorted MoE: one launch runs every row tile of one bitrate.  A row
// tile is (expert, first row, rows <= 256) of the compacted row pool; workgroup b runs column
// block b % nbn of list entry (b / nbn) / mats of matrix set (b / nbn) % mats and exits when the
// entry is past count.  No output rotation; fp16 output rows.
struct GemmGroupArgs
{
    const uint16_t* A[2];       // (pool rows, k) fp16, per matrix set
    uint16_t* C[2];             // (pool rows, n) fp16
    const uint64_t* tab[2];     // trellis address per expert
    const int* rt;              // row tiles: (expert, first row, rows) triples
    const int* list[2];         // row-tile ids at this bitrate, per matrix set
    const int* count[2];        // entries in list[i]
    int mats;                   // 1 or 2
    int k, n;
    int nrt;                    // row-tile capacity of the launch
    int tile_rows;              // rows per tile: 64, 128 or 256 (moeg: 32, 64 or 128)
    int grid_wgs;               // moeg: persistent workgroups (0: one per item)
    const float* psum[2];       // moeg, mul1: (pool rows, k / 128) chunk sums of A, per matrix set
};

int exl3k_gemm_group_k1(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_gemm_group_k2(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_gemm_group_k3(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_gemm_group_k4(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_gemm_group_k5(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_gemm_group_k6(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_gemm_group_k7(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_gemm_group_k8(const GemmGroupArgs& g, int cb, hipStream_t s);
// Register-decode grouped GEMM (exl3_gemm.hip moeg_kernel), same arguments.
int exl3k_moeg_k1(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_moeg_k2(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_moeg_k3(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_moeg_k4(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_moeg_k5(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_moeg_k6(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_moeg_k7(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_moeg_k8(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_moeg_k17(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_moeg_k18(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_moeg_k19(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_gemm_group_k17(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_gemm_group_k18(const GemmGroupArgs& g, int cb, hipStream_t s);
int exl3k_gemm_group_k19(const GemmGroupArgs& g, int cb, hipStream_t s);

// Token-sorted MoE (exl3_moe_sorted.hip).  Pool rows are the caller's temp buffers; the plan
// tables live in the library workspace.
// Rate slots of the token-sorted MoE's per (matrix, bitrate) lists: K 1..8, then 1.5 / 2.5 / 3.5.
constexpr int MOES_RATES = 11;
__host__ __device__ constexpr int moes_rate_slot(int K) { return K >= 1 && K <= 8 ? K - 1 : (K >= 17 && K <= 19 ? K - 9 : -1); }
__host__ __device__ constexpr int moes_slot_rate(int slot) { return slot < 8 ? slot + 1 : slot + 9; }

struct MoesArgs
{
    const uint16_t* x;          // (bsz, H) fp16
    float* out;                 // (bsz, H) fp32, accumulated into (atomic mode)
    float* scratch;             // (slots, H) fp32 or null: deterministic slot mode
    const int64_t* fused_base;  // slot of each expert's first row (slot mode)
    const int64_t* expert_count;    // (num_experts + 1), the last entry ignored
    const int64_t* token_sorted;    // (num_assign) token of each sorted assignment
    const uint16_t* weight_sorted;  // (num_assign) fp16 routing weight
    int num_experts, num_assign, H, I;
    int max_tokens, count_lo, count_hi;
    int pool_rows;              // rows of the temp buffers (concurrency x max_tokens)
    uint16_t *ts_g, *ts_u;      // (pool_rows, H) fp16
    uint16_t *ti_g, *ti_u;      // (pool_rows, I) fp16
    const uint64_t *g_trellis, *g_suh, *g_svh, *u_trellis, *u_suh, *u_svh, *d_trellis, *d_suh, *d_svh;
    const uint8_t *bits_g, *bits_u, *bits_d;
    int K_g, K_u, K_d;          // rate codes when there are no tables (1..8, 16 + b for b + 1/2)
    int act, gated;
    float act_limit;
    int* rowinfo;               // workspace: (sorted position or -1, expert, row within expert) per pool row
    int* rt;                    // workspace: row tiles (expert, first pool row, rows)
    int* lists;                 // workspace: 3 x MOES_RATES lists of row-tile ids, rt_cap each
    int* counts;                // workspace: 3 x MOES_RATES list lengths
    int rt_cap;
    int tile_rows;              // rows per row tile
    float *ps_g, *ps_u;         // workspace: (pool_rows, H / 128) sums of each staged 128-chunk
    float* ps_d;                // workspace: (pool_rows, I / 128) the same for the down input
    // token-major output (atomic mode): per-token lists of sorted positions and, per pass, the
    // pool row of each position
    int bsz;                    // tokens (rows of x and out)
    int* tok_start;             // workspace: (bsz + 1) list starts
    int* tok_pos;               // workspace: (num_assign) sorted positions, ascending per token
    int* inv_row;               // workspace: (num_assign) pool row of a position in the current pass
};

struct MoesGatherArgs
{
    float* out;                 // (tokens, H) fp32
    const float* scratch;       // (slots, H) fp32
    const int64_t *flat_expert, *inv_order, *expert_start, *slot_base, *slot_kind;
    const uint16_t* weight_sorted;
    int tokens, H, topk, num_experts;
};

int exl3k_rms_norm_res(const uint16_t* x, const uint16_t* r, const uint16_t* w, uint16_t* y, uint16_t* n,
                       long rows, int dim, float eps, hipStream_t s);
// Most chunk sums of squares one lane of the split norm's consumer loads: rows of at most
// 64 * 4 * 128 = 32768 columns.
constexpr int SQ_SCALE_MAX_PER_LANE = 4;

// Split residual norm, standalone halves (exl3_decode_ops.hip): h = fp16(h + c) with per-chunk
// sums of squares (c null: h unchanged), and r = fp16(fp16(h * scale) * w) from those sums.
int exl3k_res_sq(uint16_t* h, const uint16_t* c, float* sq, long rows, int n, hipStream_t s);
int exl3k_norm_sq(const uint16_t* h, const float* sq, const uint16_t* w, uint16_t* r, long rows, int n, float eps,
                  hipStream_t s);
int exl3k_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* out, long n, hipStream_t s);

int exl3k_moes_plan(const MoesArgs& a, int pass_row0, hipStream_t s);
int exl3k_moes_gather(const MoesArgs& a, int cus, hipStream_t s);
int exl3k_moes_act(const MoesArgs& a, int cus, hipStream_t s);
int exl3k_moes_out(const MoesArgs& a, int cus, hipStream_t s);
int exl3k_moes_tokens(const MoesArgs& a, hipStream_t s);
size_t exl3k_moes_tokens_lds(int bsz, int num_assign);       // bytes; at most 160 KiB
int exl3k_moes_sum(const MoesGatherArgs& a, hipStream_t s);

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
    XcdGuard xg;                // hand-off check (used when xcd > 0)
    int run_lo, run_hi;         // this launch takes the runs of run_lo + 1 .. run_hi slots
    int epi_serial;             // 1: the gate/up and down epilogues' general loops (test policy)
};

int exl3k_moe_cb0(const MoeArgs& a, hipStream_t s);
int exl3k_moe_cb1(const MoeArgs& a, hipStream_t s);
int exl3k_moe_cb2(const MoeArgs& a, hipStream_t s);
constexpr int EXL3_MOE_SBMAX = 64;     // k-slices per workgroup of the MoE GEMV (LDS bound)

int exl3k_reconstruct(uint16_t* W, const uint16_t* trellis, int k, int n, int tiles_n,
                      int nt_off, int K, int cb, hipStream_t s);
int exl3k_reconstruct_tr(uint16_t* WT, const uint16_t* trellis, int k, int n, int tiles_n,
                         int nt_off, int K, int cb, const uint16_t* svh, int slabs, hipStream_t s);
int exl3k_reconstruct_had(uint16_t* W, const uint16_t* trellis, const uint16_t* suh,
                          const uint16_t* svh, int k, int n, int tiles_n, int nt_off,
                          int K, int cb, hipStream_t s);

int exl3k_xcd_probe(int* out, int blocks_x, int blocks_y, hipStream_t s);
int exl3k_fill_u32(uint32_t* p, uint32_t v, size_t n, hipStream_t s);
int exl3k_mgemm_filter(const int64_t* indices, const uint16_t* weights, int bszm, int min_index,
                       int max_index, int num_tokens, int64_t* idx_out, uint16_t* w_out, hipStream_t s);

// reconstruct_had written transposed: WT (n, k)
int exl3k_reconstruct_had_tr(uint16_t* WT, const uint16_t* trellis, const uint16_t* suh,
                             const uint16_t* svh, int k, int n, int tiles_n, int nt_off,
                             int K, int cb, int slabs, hipStream_t s);
// Dense fp16 GEMM C (m, n) = A (m, k) . WT (n, k)^T, fp32 accumulation; svh non-null: output
// rotation per 128-column chunk, x svh (exl3_dense.hip)
int exl3k_split_fixup(const float* part, void* C, const uint16_t* svh, int m, int n, int ldc, int c_fp32, int nmb,
                      int tiles, int splits, hipStream_t s);
int exl3k_dense_gemm(const uint16_t* A, const uint16_t* WT, void* C, int c_fp32, const uint16_t* svh,
                     int m, int k, int n, int a_slabs, int w_slabs, int ldc, int variant, int cus,
                     float* part, size_t part_bytes, hipStream_t s);
int exl3k_had128(const void* in, void* out, int rows, int cols, int fp32,
                 const uint16_t* pre, const uint16_t* post, float scale, int slabs, hipStream_t s);
int exl3k_slab_copy(const uint16_t* x, uint16_t* y, int rows, int cols, hipStream_t s);

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
