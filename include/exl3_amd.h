/*
 * exl3_amd.h -- C ABI of the MI355X (gfx950) EXL3 quantized-linear library (libexl3_amd.so).
 *
 * Plain pointers and sizes only; no torch or C++ types cross this boundary.  Every entry
 * point validates its arguments before launching anything, returns 0 (or a non-negative
 * kernel tag) on success and a negative EXL3_AMD_E* code on failure, never throws, and
 * enqueues its work on `stream` (a hipStream_t; NULL = the default stream) without host
 * synchronisation, so the calls are graph-capturable once the device is initialised.
 * exl3_amd_last_error() returns the message of the calling thread's last failure.
 *
 * Data layout (the reference's, unchanged):
 *   trellis  uint16 (k/16, n/16, 16*K) row-major, K = bits per weight (1..8)
 *   suh      fp16 (k) input sign/scale vector;  svh fp16 (n) output vector
 *   A / x    fp16 (m, k) row-major;  C / y fp16 or fp32 (m, n) row-major
 *   W        fp16 (k, n) row-major, y = x @ W (no transpose)
 * Codebook: mcg = 1 selects MCG, mul1 = 1 selects MUL1, neither = 3INST (not both).
 *
 * Each entry point names the reference interface it replaces (file:line, paths relative to
 * the jow-/ampstein tree; vendor/exl3 = exllamav3 v1.5.3 @ d3739fd).
 */
#ifndef EXL3_AMD_H
#define EXL3_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EXL3_AMD_OK            0
#define EXL3_AMD_EINVAL       -1   /* bad argument: shape, bitrate, null pointer, codebook  */
#define EXL3_AMD_EUNSUPPORTED -2   /* valid reference input this build does not implement  */
#define EXL3_AMD_EHIP         -3   /* HIP runtime error                                     */
#define EXL3_AMD_ENOMEM       -4   /* workspace allocation failed                           */

/* Kernel tags returned by exl3_amd_gemm (the reference returns a shape index, 90 = GEMV). */
#define EXL3_AMD_TAG_GEMV     90
#define EXL3_AMD_TAG_GEMM     91

/* Thread-local message of the last failing call ("" if none). */
const char* exl3_amd_last_error(void);

/* Library ABI version (major * 10000 + minor * 100 + patch). */
int exl3_amd_version(void);

/* Kernel-path policy, process-wide.  Every key defaults to 0, the library's own choice (the
 * measured fastest path for the shape).  A nonzero value selects an alternative kernel path that
 * computes the same result, so that tests can cover every instance and benchmarks can compare
 * paths.  Calls made while another thread changes a policy see either value.  No counterpart in
 * the reference (its tuning is compiled in); for tests and benchmarks. */
#define EXL3_AMD_POLICY_GEMV_ROWS       0   /* rows of the GEMV (exl3_gemm / exl3_mgemm, m <= 16)       */
#define EXL3_AMD_GEMV_ROWS_LDS          1   /*   the LDS kernel for 2..8 rows, no matrix-core GEMV      */
#define EXL3_AMD_GEMV_ROWS_MFMA_ALL     2   /*   the matrix-core GEMV for single rows as well           */
#define EXL3_AMD_POLICY_GEMM_STAGING    1   /* operand staging of the fused MFMA GEMM (m > 8)          */
#define EXL3_AMD_GEMM_STAGING_REGS      1   /*   register-staged instead of LDS DMA                     */
#define EXL3_AMD_GEMM_STAGING_NO_SPLIT  2   /*   LDS DMA without the split k of launches whose tiles
                                                 fill at most half the CUs                              */
#define EXL3_AMD_POLICY_MOE_GEMM        2   /* grouped GEMM of exl3_amd_moe                            */
#define EXL3_AMD_MOE_GEMM_LDS           1   /*   the LDS-tiled kernel instead of the register decode    */
#define EXL3_AMD_POLICY_MOE_TILE_ROWS   3   /* exl3_amd_moe row-tile height: 0 = by mean rows, else the
                                             * value (32 / 64 / 96 / 128; LDS-tiled: 64 / 128 / 256)  */
#define EXL3_AMD_POLICY_MOE_OUTPUT      4   /* exl3_amd_moe output kernel                              */
#define EXL3_AMD_MOE_OUTPUT_ATOMIC      1   /*   per-row atomics instead of the per-token lists         */
#define EXL3_AMD_POLICY_RECON_MM        5   /* kernel of exl3_amd_recon_mm                             */
#define EXL3_AMD_RECON_MM_8WAVES        1   /*   8 waves of 128 x 64 instead of 4 waves of 128 x 128    */
#define EXL3_AMD_RECON_MM_WHOLE_TILES   2   /*   four-wave form without half tiles in a last round      */
#define EXL3_AMD_RECON_MM_GLOBAL_DMA    3   /*   four-wave form, DMAs on 64-bit lane addresses (the form
                                                 used for operands of 4 GiB and more)                   */
#define EXL3_AMD_RECON_MM_NO_SPLIT      5   /*   four-wave form without the split k of launches whose
                                                 tiles fill at most half the CUs                        */
#define EXL3_AMD_POLICY_GEMV_SPLIT      6   /* work split of the single-row GEMV                       */
#define EXL3_AMD_GEMV_SPLIT_BALANCED    1   /*   equal work per wave and waves per SIMD (gemv1b_kernel)  */
#define EXL3_AMD_POLICY_GEMV_SLICES     7   /* single-row stream GEMV: k-slices per workgroup (0 = by the
                                             * planner; a valid forced value: 4, 8, 16 or a multiple of 32
                                             * dividing k / 16)                                        */
#define EXL3_AMD_POLICY_XCD_FAKE        8   /* test hook of the XCD hand-off check: value v > 0 makes
                                             * linear workgroup v - 1 of every hand-off launch report
                                             * XCC id + 1, as if dispatch had put it on another XCD   */
#define EXL3_AMD_POLICY_MOE_EPILOGUE    9   /* exl3_amd_moe_coop gate/up and down epilogues            */
#define EXL3_AMD_MOE_EPILOGUE_SERIAL    1   /*   their general loops, each load consumed as it arrives,
                                                 instead of the forms that issue every load first
                                                 (gate/up: at most 4 k-splits; down: top-k <= 16, at
                                                 most 2 k-splits); same bits                            */
#define EXL3_AMD_POLICY_COUNT           10
int exl3_amd_set_policy(int key, int value);
int exl3_amd_get_policy(int key);       /* the current value, or EXL3_AMD_EINVAL for an unknown key */

/* Allocate the per-device workspace (split-k partials and completion counters) of `device`.
 * Optional: the first call on a device does it lazily.  Call it before capturing a graph.
 * Replaces DevCtx::get_locks (vendor/exl3/exllamav3_ext/quant/exl3_devctx.cu:81-93). */
int exl3_amd_init(int device);

/* Topology the library planned for on `device` (initialising it if needed): compute units and
 * the number of XCDs whose round-robin workgroup dispatch was verified on the device (0: the
 * XCD-local split-k hand-off is off and a finish kernel sums the partials).  No counterpart in
 * the reference; for tests and benchmarks. */
int exl3_amd_device_info(int device, int* num_cus, int* num_xcd);

/* Per-launch check of the XCD-local split-k hand-off (no counterpart in the reference).  Every
 * hand-off counter also sums its arrivals' XCC ids and their squares; the last arrival sets the
 * device's alarm (pinned host memory) when the ids differ, i.e. when dispatch put workgroups of
 * one counter on two XCDs.  Every call reads the alarm first: once it is set, the library turns
 * the hand-off off for the device (num_xcd 0, the finish kernel and agent-scope hand-offs take
 * over), zeroes the counters, and reports on stderr.  Outputs of the launch that raised the alarm
 * are not reliable.
 * xcd_status synchronises the device, services the alarm and reports the probe's XCD count, the
 * count in use and the alarms seen so far.  xcd_rearm (tests) clears the alarm and restores the
 * probe's count.  For tests and monitoring. */
int exl3_amd_xcd_status(int device, int* probe_xcd, int* active_xcd, int* alarms);
int exl3_amd_xcd_rearm(int device);

/* Host-side view of the hand-off's workgroup mapping (the kernels' own functions; no device
 * needed): kind 0, GEMV split grid (p0 splits): out = { chunk, slot }; kind 1, MoE stage grid
 * (p0 chunks): out = { chunk, rest }; kind 2, balanced single-row stream (p0 pairs, p1 k / 16,
 * p2 slices per wave): out = { valid, pair A, pair B, straddles }; kind 3, its pair span (p1, p2,
 * b = pair position q): out = { first local index, count }.  No counterpart in the reference;
 * for the CPU test of the mapping. */
int exl3_amd_debug_handoff_map(int kind, int xcd, int p0, int p1, int p2, int b, int* out);

/* Test hooks (no counterpart in the reference).  The per-device workspace holds split-k
 * partials and, during exl3_amd_moe, the token-sorted MoE's plan (row map, row tiles, tile lists,
 * chunk sums, per-token position lists).  read_workspace copies `bytes` from byte `offset` of it
 * to host memory; fill_workspace sets every byte of it (e.g. 0xff: int -1, fp32 NaN) so that a
 * test can show that a call reads nothing it did not write.  Both synchronise the device; neither
 * may be called while work that uses the workspace is being captured. */
int exl3_amd_debug_read_workspace(int device, int64_t offset, int64_t bytes, void* host_dst);
int exl3_amd_debug_fill_workspace(int device, int byte_value);

/* W_hat (k, n) fp16 = decoded trellis columns [n_offset, n_offset + n) of a packed tensor
 * whose full width is n_packed, in the Hadamard basis.  k % 16 == 0, n % 128 == 0,
 * n_offset % 128 == 0.  Bit-exact with the reference.
 * Replaces reconstruct / reconstruct_slice (vendor/exl3/exllamav3_ext/quant/reconstruct.cu:141-208,
 * :492-501), bound at src/torch/amp_torch.cpp:11016-11057 (torch.exl3_reconstruct). */
int exl3_amd_reconstruct(uint16_t* W, const uint16_t* trellis, int k, int n_packed, int n,
                         int n_offset, float K, int mcg, int mul1, void* stream);

/* W_hat transposed: WT (n, k) fp16 row-major, WT[c][r] = W_hat[r][c] for the columns
 * [n_offset, n_offset + n) of the packed tensor; same arguments and validation as
 * exl3_amd_reconstruct, bit-exact values.  No counterpart in the reference (whose recon path
 * stores W (k, n) for cuBLAS, amp_torch.cpp:11199-11214): the layout in which the recon GEMM
 * (exl3_gemm_recon) reads both operands k-contiguous. */
int exl3_amd_reconstruct_t(uint16_t* WT, const uint16_t* trellis, int k, int n_packed, int n,
                           int n_offset, float K, int mcg, int mul1, void* stream);

/* W (k, n) fp16 = diag(suh) . H128 . W_hat . H128 . diag(svh) per 128x128 block (original
 * basis), bit-exact with the reference's fp16 rounding.  k, n, n_offset multiples of 128;
 * suh has k entries, svh has n entries (pre-offset by the caller for a slice).
 * Replaces reconstruct_had_slice (vendor/exl3/exllamav3_ext/quant/reconstruct.cu:431-490),
 * declared at src/torch/amp_torch.cpp:11068-11078. */
int exl3_amd_reconstruct_had(uint16_t* W, const uint16_t* trellis, const uint16_t* suh,
                             const uint16_t* svh, int k, int n_packed, int n, int n_offset,
                             float K, int mcg, int mul1, void* stream);

/* y = H128(x (o pre)) * scale / sqrt(128) (o post) over each 128-column chunk of each row.
 * fp32 = 0: x, y fp16; fp32 = 1: x, y fp32.  pre / post fp16 (cols) or NULL; at most one
 * of them may be given.  In place (x == y) allowed.  cols % 128 == 0.
 * Replaces had_r_128 (vendor/exl3/exllamav3_ext/quant/hadamard.cu:125-210), declared at
 * src/torch/amp_torch.cpp:11060-11066. */
int exl3_amd_had_r_128(const void* x, void* y, int rows, int cols, int fp32,
                       const uint16_t* pre, const uint16_t* post, float scale, void* stream);

/* C (m, n) = had(had(A o suh) @ W_hat) o svh, C fp16 (c_fp32 = 0) or fp32.  suh / svh may be
 * NULL (that rotation is skipped).  A_had: caller scratch of A's shape, accepted for interface
 * parity and not written (the rotation is recomputed per workgroup).  k % 128 == 0 and
 * n % 128 == 0 when a rotation is requested, else k % 16 and n % 128.  Returns a kernel tag.
 * force_shape_idx > 0 forces a kernel (1 = GEMV, 2 = MFMA GEMM); <= 0 = by shape.
 * K: 1..8, or 1.5 / 2.5 / 3.5 with mul1; at a half rate more than 8 rows run the GEMV in
 * row groups of 8 (tag 90).
 * Replaces exl3_gemm (vendor/exl3/exllamav3_ext/quant/exl3_gemm.cu:321-350, dispatcher
 * :114-319), bound at src/torch/amp_torch.cpp:11251-11294 (torch.exl3_gemm). */
int exl3_amd_gemm(const uint16_t* A, const uint16_t* trellis, void* C, int c_fp32,
                  const uint16_t* suh, uint16_t* A_had, const uint16_t* svh,
                  int m, int k, int n, float K, int mcg, int mul1, int force_shape_idx,
                  void* stream);

/* exl3_amd_gemm without any allocation: the same operation, arguments, kernels and error codes,
 * but the GEMV's split-k partials (and the MFMA GEMM's partial tiles when it splits k, with no
 * more splits than 16 MiB holds), completion counters and prefetch sink live in a file-scope
 * device array of the library (16 MiB of partials, 256 KiB of counters, 8 KiB sink) instead of
 * the workspace exl3_amd_gemm allocates on first use.  It calls no hipMalloc / hipFree and no
 * allocating library routine, so it serves callers that cannot allocate (code under stream
 * capture, serving loops, harnesses that forbid allocation).  A shape whose split partials
 * exceed the array returns EXL3_AMD_EUNSUPPORTED with a message.  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (concurrent streams) race.  Call
 * exl3_amd_init(device) first to take the XCD-local hand-off; without it the partials are
 * summed by a second kernel.
 * No counterpart in the reference: an entry point of this build for the callers that cannot
 * allocate. */
int exl3_amd_gemm_noalloc(const uint16_t* A, const uint16_t* trellis, void* C, int c_fp32,
                          const uint16_t* suh, uint16_t* A_had, const uint16_t* svh,
                          int m, int k, int n, float K, int mcg, int mul1, int force_shape_idx,
                          void* stream);

/* Multi-matrix GEMV over device pointer tables: slot j (0 <= j < max(bszm_in, bszm_out))
 * computes C[j] = had(had(A[j or 0] o suh[q]) @ W_hat[q]) o svh[q] with q = indices[j] (or j;
 * negative = slot skipped).  Tables B, suh, svh hold num_B device addresses (uint64) of
 * trellis (k/16, n/16, 16K) uint16, suh (k) fp16 and svh (n) fp16.  A (bszm_in, m, k) fp16;
 * C (bszm_out, m, n) fp16 / fp32.
 *   weights (fp16 per slot): every output is scaled by its weight, then the slots of each of
 *     num_tokens groups (bszm / num_tokens consecutive slots) are summed into C[t].
 *   min_index >= 0: selections outside [min_index, max_index) dropped (one token: compacted,
 *     several: masked), kept ones rebased by min_index (at most 128 slots).
 *   size_n_list + c_ptrs (num_c_ptrs entries): per-matrix width and output address.
 *   sliced mode (had_src_list, n_stride_list, num_had_src): entries are equal-width column
 *     slices of num_had_src source matrices; B / svh / c_ptrs pre-offset to the slice, the row
 *     stride of trellis tiles and C is n_stride_list[q], suh is per source had_src_list[q].
 * All tables and lists are device memory.  A_had: scratch of had_slabs * m * k elements
 * (checked, not written).  k % 128 == 0; n % 128 == 0.  More than 8 rows run as row groups
 * of 8 (not with weights).
 * Replaces exl3_mgemm (vendor/exl3/exllamav3_ext/quant/exl3_gemm.cu:396-712, semantics
 * :352-394, kernel exl3_gemm_kernel.cuh:88-343), declared at src/torch/amp_torch.cpp:3841-3864
 * and bound at :10194-10330 (torch.mgemm). */
int exl3_amd_mgemm(const uint16_t* A, int bszm_in, int m, int k,
                   const uint64_t* B, int num_B,
                   void* C, int bszm_out, int n, int c_fp32,
                   const uint64_t* suh, int num_suh,
                   uint16_t* A_had, int64_t a_had_numel,
                   const uint64_t* svh, int num_svh,
                   const int64_t* indices, int num_indices,
                   const uint16_t* weights,
                   float K, int force_shape_idx, int mcg, int mul1,
                   int min_index, int max_index, int force_num_sms, int num_tokens,
                   const int* size_n_list, const uint64_t* c_ptrs, int num_c_ptrs,
                   const int* n_stride_list, int num_n_stride,
                   const int* had_src_list, int num_had_src_list, int num_had_src,
                   void* stream);

/* Fused decode-shaped MoE: out[t] = sum over token t's active slots k (expert e = sel[t, k],
 * rw[t, k] != 0, inside [min_expert, max_expert) when min_expert >= 0) of
 * rw[t, k] * down_e(act(gate_e(x_t), up_e(x_t))) (+ sigmoid-gated shared expert sh_out).
 * Tables (n_local entries of device addresses): g/u/d trellis, suh, svh (+ optional bias);
 * bits_g/u/d (uint8 per expert, mul1 only) select mixed widths, else Kg = Ku, Kd.  act: 0 SiLU,
 * 1 GELU, 2 ReLU^2, 3 clamped SwiGLU; gated = 0: act = relu(u) * u.  Scratch: had_g / had_u
 * (slots, Hi) fp16, act_out (slots, I) fp16, d_out (slots, Ho) fp32, gu_g / gu_u (slots, I)
 * (sizes checked; the library keeps its split partials in its own workspace), ctr int32 of at
 * least slots_max * I/128 + rows_max * Ho/128 + 2 + 2 * slots_max + 1 entries: the run table
 * (active slots sorted by (expert, slot), runs of <= 8) is written at offset
 * slots_max * I/128 + rows_max * Ho/128.  out fp32 (rows_max, H_out) row stride out_stride.
 * Replaces exl3_moe_coop (vendor/exl3/exllamav3_ext/quant/exl3_moe_coop.cu:185-371, kernels
 * exl3_moe_coop_kernel.cuh:231-1000), declared at src/torch/amp_torch.cpp:7783-7837 and bound
 * at :7853 (torch.moe_coop). */
int exl3_amd_moe_coop(const uint16_t* x, int bsz, int H, int x_stride,
                      const int64_t* sel, const uint16_t* rw, int topk,
                      int min_expert, int max_expert, int Hi,
                      const uint64_t* g_trellis, const uint64_t* g_suh, const uint64_t* g_svh,
                      const uint64_t* u_trellis, const uint64_t* u_suh, const uint64_t* u_svh,
                      const uint64_t* d_trellis, const uint64_t* d_suh, const uint64_t* d_svh, int n_local,
                      const uint64_t* g_bias, const uint64_t* u_bias, const uint64_t* d_bias,
                      float Kg, float Ku, float Kd, int mcg, int mul1, int act, float act_limit, int gated,
                      uint16_t* had_g, int64_t had_g_numel, uint16_t* had_u, int64_t had_u_numel,
                      void* gu_g, void* gu_u, int64_t gu_numel, int gu_f32, int I,
                      uint16_t* act_out, int64_t act_out_numel, float* d_out, int64_t d_out_numel, int Ho,
                      int* ctr, int64_t ctr_numel,
                      float* out, int rows_max, int H_out, int out_stride,
                      const float* sh_out, const uint16_t* sh_gate_w, int sh_gate_n,
                      const uint8_t* bits_g, const uint8_t* bits_u, const uint8_t* bits_d,
                      void* stream);

/* Workgroup groups the reference's token-sorted MoE would run on this device (num_cus / 8): the
 * caller sizes the temp buffers' first dimension with it.  Replaces exl3_moe_max_concurrency
 * (vendor/exl3/exllamav3_ext/quant/exl3_moe.cu:15-19).  Returns >= 0, or a negative error code. */
int exl3_amd_moe_max_concurrency(int device);

/* Token-sorted fused MoE for prefill-sized batches.  For every expert e whose token count c
 * (expert_count[e], expert_count_len = num_experts + 1, last entry ignored) satisfies
 * 0 < c <= max_tokens_per_expert and count_lo <= c <= count_hi, and every one of its
 * assignments (token_sorted / weight_sorted, sorted by expert, num_assign = bsz * top-k):
 *     y = w * (had(down_e(had(act(had(gate_e(h)) o svh_g, had(up_e(h)) o svh_u) o suh_d))) o svh_d)
 * with h = had(x[token] o suh_g / suh_u), is added atomically to output_state[token] (fp32,
 * (bsz, hidden_dim)), or, with output_scratch (scratch_rows x scratch_cols fp32) and fused_base
 * (int64 per expert), stored in slot fused_base[e] + (row of the assignment within e).
 * act_function: 0 SiLU, 1 GELU, 2 non-gated ReLU^2 (gate skipped), else identity; act_limit != 0
 * clamps.  Temp buffers: temp_state_g / _u (concurrency, max_tokens_per_expert, hidden_dim) fp16,
 * temp_intermediate_g / _u (concurrency, max_tokens_per_expert, intermediate_dim) fp16, used as
 * one pool of rows (more routed rows than the pool holds run in passes).  mcg or mul1 codebook;
 * bits_g/u/d (uint8 per expert, mul1) select per-expert integer widths.  Unlike the reference,
 * every in-range expert runs in one set of launches (no group barriers); half-integer rates
 * return EXL3_AMD_EUNSUPPORTED.
 * Replaces exl3_moe (vendor/exl3/exllamav3_ext/quant/exl3_moe.cu:137-418, kernel
 * exl3_moe_kernel.cuh:78-313), declared at src/torch/amp_torch.cpp:7796-7837 and bound at :9269
 * (torch.moe_fused). */
int exl3_amd_moe(const uint16_t* hidden_state, int bsz, int hidden_dim, float* output_state,
                 const int64_t* expert_count, int expert_count_len,
                 const int64_t* token_sorted, const uint16_t* weight_sorted, int num_assign,
                 uint16_t* temp_state_g, uint16_t* temp_state_u, int concurrency, int max_tokens_per_expert,
                 uint16_t* temp_intermediate_g, uint16_t* temp_intermediate_u, int intermediate_dim,
                 int act_function, float K_gate, float K_up, float K_down,
                 const uint64_t* gate_ptrs_trellis, const uint64_t* gate_ptrs_suh, const uint64_t* gate_ptrs_svh,
                 const uint64_t* up_ptrs_trellis, const uint64_t* up_ptrs_suh, const uint64_t* up_ptrs_svh,
                 const uint64_t* down_ptrs_trellis, const uint64_t* down_ptrs_suh, const uint64_t* down_ptrs_svh,
                 int num_ptrs,
                 int gate_mcg, int gate_mul1, int up_mcg, int up_mul1, int down_mcg, int down_mul1,
                 float act_limit, int num_active,
                 float* output_scratch, int64_t scratch_rows, int scratch_cols, const int64_t* fused_base,
                 int count_lo, int count_hi, int m_tile,
                 const uint8_t* bits_g, const uint8_t* bits_u, const uint8_t* bits_d, int bits_len,
                 void* stream);

/* Fixed-order reduction of exl3_amd_moe's slots: for every token, output_state[token] +=
 * sum over its top-k assignments a (in k order) of output_scratch[slot(a)] * wt(a), with
 * e = flat_expert[a], slot = slot_base[e] + inv_order[a] - expert_start[e] when slot_kind[e]
 * != 0 (kind 2: wt = weight_sorted[inv_order[a]], else 1).  top-k <= 32.
 * Replaces exl3_moe_gather (vendor/exl3/exllamav3_ext/quant/exl3_moe.cu:420-531), declared at
 * src/torch/amp_torch.cpp:7783-7794 and bound at :9359 (torch.moe_gather). */
int exl3_amd_moe_gather(float* output_state, int tokens, int hidden_dim,
                        const float* output_scratch, int scratch_cols,
                        const int64_t* flat_expert, int num_assign, const int64_t* inv_order,
                        const int64_t* expert_start, int expert_start_len,
                        const int64_t* slot_base, int slot_base_len,
                        const int64_t* slot_kind, int num_experts,
                        const uint16_t* weight_sorted, void* stream);

/* Fused residual add + RMSNorm over rows of dim (a multiple of 4) fp16 values:
 * y = fp16(x + r) (the updated residual stream; y may alias x),
 * n = fp16(fp16(y * rsqrt(mean(y^2) + eps)) * w).  Pointers 8-byte aligned.
 * Replaces amp_rms_norm_res_fp16 (src/torch/amp_kernels.cu:367-397, kernel :279-365), bound at
 * src/torch/amp_torch.cpp:10081 (torch.rms_norm_res). */
int exl3_amd_rms_norm_res(const uint16_t* x, const uint16_t* r, const uint16_t* w, uint16_t* y, uint16_t* n,
                          int64_t rows, int dim, float eps, void* stream);

/* out = fp16(silu(g) * u) elementwise, fp32 math.  Replaces amp_silu_mul_fp16
 * (src/torch/amp_kernels.cu:253-268, kernel :235-251), bound at src/torch/amp_torch.cpp:4966
 * (torch.silu_mul). */
int exl3_amd_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* out, int64_t numel, void* stream);

/* C = exl3_gemm(silu(gate) * up) in one call: the decode step's SwiGLU + down projection
 * (graphdec.uc:206-217 calls torch.silu_mul, then torch.exl3_gemm).  With one row the M = 1
 * stream kernel forms silu(gate) * up, rounded to fp16 as silu_mul does, while loading its input
 * (one launch, act untouched); otherwise silu_mul writes act (m, k) and exl3_gemm reads it.
 * Same results as the two calls.  No counterpart in the reference (a fusion of two of its calls).
 * Returns the exl3_gemm tag. */
int exl3_amd_gemm_silu_mul(const uint16_t* gate, const uint16_t* up, uint16_t* act,
                           const uint16_t* trellis, void* C, int c_fp32,
                           const uint16_t* suh, uint16_t* A_had, const uint16_t* svh,
                           int m, int k, int n, float K, int mcg, int mul1, void* stream);

/* The decode step's linear + residual norm in one call (graphdec.uc:184-189 and :223 then the
 * next norm): C = exl3_gemm(A) (or of fp16(silu(A) * up) when up is given, with act as the
 * fallback's scratch), then h = fp16(h + C) in place and r = fp16(fp16(h * rsqrt(mean(h^2) +
 * eps)) * w), like exl3_amd_rms_norm_res.  With one row, the M = 1 stream GEMV does the norm in
 * the wave that completes the row's last column chunk: one launch.  Otherwise (or without the
 * XCD hand-off) the GEMM and exl3_amd_rms_norm_res run as two launches.  C fp16; C, h, w, r
 * 16-byte aligned.  No counterpart in the reference (a fusion of two of its calls).  Returns the
 * exl3_gemm tag. */
int exl3_amd_gemm_norm(const uint16_t* A, const uint16_t* up, uint16_t* act, const uint16_t* trellis, uint16_t* C,
                       const uint16_t* suh, uint16_t* A_had, const uint16_t* svh,
                       int m, int k, int n, float K, int mcg, int mul1,
                       uint16_t* h, const uint16_t* w, uint16_t* r, float eps, void* stream);

/* The decode step's residual norm (rms_norm_res, src/torch/amp_kernels.cu:279-365, bound at
 * src/torch/amp_torch.cpp:10081, called between the linears at graphdec.uc:151-230) split
 * between its two neighbours, so that the norm costs no launch and no serial pass of its own.
 * A row of n columns is handled in 128-column chunks; sq holds one fp32 per chunk (rows x n/128):
 *   producer   h = fp16(h + c), sq[chunk] = sum over the chunk of float(h)^2
 *              (exl3_amd_gemm_res in the GEMV's epilogue; exl3_amd_res_sq on its own);
 *   consumer   r = fp16(fp16(h * scale) * w), scale = 1 / sqrtf(sum(sq) / n + eps), the chunk
 *              sums added in a fixed order (exl3_amd_mgemm_norm_in in the GEMV's input load;
 *              exl3_amd_norm_sq on its own).
 * h and r are exactly rms_norm_res's y and n except for the order in which the sum of squares
 * is accumulated (r within one fp16 ulp); the fused and standalone forms of each half give the
 * same bits.  No counterpart in the reference (a re-division of its rms_norm_res).  n <= 32768
 * for the consumer.  Pointers 4-byte aligned.  Returns 0 or a negative error. */
int exl3_amd_res_sq(uint16_t* h, const uint16_t* c, float* sq, int rows, int n, void* stream);
int exl3_amd_norm_sq(const uint16_t* h, const float* sq, const uint16_t* w, uint16_t* r, int rows, int n, float eps,
                     void* stream);

/* exl3_gemm (or, with up, exl3_amd_gemm_silu_mul) followed by the producer half of the split
 * residual norm: C = the linear (fp16), h = fp16(h + C), sq = its chunk sums.  With one row the
 * GEMV's chunk epilogue does the residual add and the sums: one launch.  Otherwise two (the
 * linear, then exl3_amd_res_sq).  Returns the exl3_gemm tag. */
int exl3_amd_gemm_res(const uint16_t* A, const uint16_t* up, uint16_t* act, const uint16_t* trellis, uint16_t* C,
                      const uint16_t* suh, uint16_t* A_had, const uint16_t* svh,
                      int m, int k, int n, float K, int mcg, int mul1,
                      uint16_t* h, float* sq, void* stream);

/* exl3_amd_mgemm of the consumer half of the split residual norm: the input is rmsnorm(h) * w
 * formed from h and its chunk sums sq (k / 128 per row), as exl3_amd_norm_sq writes it.  Stacked
 * (one input slab broadcast to num_B matrices) or sliced mode (size_n_list .. num_had_src as in
 * exl3_amd_mgemm); no indices, routing weights or token groups.  With one row the M = 1 stream
 * GEMV normalises its input chunks while loading them (one launch; every wave forms the scale
 * from the same sums in the same order); otherwise exl3_amd_norm_sq writes r (m, k) first and
 * the GEMV reads it.  Results bit-identical to exl3_amd_norm_sq followed by exl3_amd_mgemm on r.
 * No counterpart in the reference.  Returns the exl3_mgemm tag. */
int exl3_amd_mgemm_norm_in(const uint16_t* h, int bszm_in, int m, int k,
                           const uint64_t* B, int num_B,
                           void* C, int bszm_out, int n, int c_fp32,
                           const uint64_t* suh, int num_suh,
                           uint16_t* A_had, int64_t a_had_numel,
                           const uint64_t* svh, int num_svh,
                           const int* size_n_list, const uint64_t* c_ptrs, int num_c_ptrs,
                           const int* n_stride_list, int num_n_stride,
                           const int* had_src_list, int num_had_src_list, int num_had_src,
                           float K, int mcg, int mul1,
                           const float* sq, const uint16_t* w, float eps, uint16_t* r,
                           void* stream);

/* exl3_amd_reconstruct_had written transposed: WT (n, k) row-major, WT[c][r] = W[r][c], the same
 * fp16 values bit for bit.  The layout exl3_amd_recon_mm reads.  No counterpart in the reference
 * (reconstruct_had_slice, quant/reconstruct.cu:431-490, writes (k, n) for cuBLAS); the recon
 * route's many-rows branch (src/torch/amp_torch.cpp:11203-11209) uses it. */
int exl3_amd_reconstruct_had_t(uint16_t* WT, const uint16_t* trellis, const uint16_t* suh,
                               const uint16_t* svh, int k, int n_packed, int n, int n_offset,
                               float K, int mcg, int mul1, void* stream);

/* Dense fp16 GEMM of the recon route: C (m, n) = A (m, k) . WT^T with the weight stored transposed,
 * WT (n, k) row-major; fp32 accumulation; C fp32 (c_fp32) or fp16.  svh non-null: each 128-column
 * chunk of the fp32 row is rotated (H128 / sqrt(128)) and multiplied by svh before the store (the
 * rotated branch's output rotation).  k % 32 == 0, n % 128 == 0, any m.  Hand-written MFMA kernel
 * (exl3_dense.hip); launches whose 256 x 256 tiles fill at most half the CUs split k, with the
 * partial tiles in the library workspace (the first call on a device allocates it, like the
 * GEMV's).  Replaces the cuBLAS GEMM of the recon route (src/torch/amp_torch.cpp:11083-11230). */
int exl3_amd_recon_mm(const uint16_t* A, const uint16_t* WT, void* C, int c_fp32, const uint16_t* svh,
                      int m, int k, int n, void* stream);

/* exl3_amd_reconstruct_t with the output rotation folded in: WT (n, k) = (W_hat H128 diag(svh)
 * / sqrt(128))^T for columns [n_offset, n_offset + n), svh the full (n_packed) vector.  fp32
 * butterflies from the fp16 weights, one fp16 rounding.  The recon GEMM's rotated branch then
 * computes y = had(x o suh) @ W' with no rotation of y.  No counterpart in the reference (its
 * rotated branch rotates y, amp_torch.cpp:11215-11228). */
int exl3_amd_reconstruct_t_had(uint16_t* WT, const uint16_t* trellis, const uint16_t* svh, int k, int n_packed,
                               int n, int n_offset, float K, int mcg, int mul1, void* stream);

/* The k-slab layout of a (rows, k) fp16 operand: element (r, c) at (c / 32) * rows * 32 + r * 32
 * + c % 32, i.e. k / 32 slabs, each the 64 bytes of every row for 32 consecutive k.  One k stage
 * of the dense GEMM is then one contiguous slab, and each of its LDS DMAs reads a contiguous
 * kilobyte (8 whole cache lines) instead of 64 bytes of 16 rows; measured ~6 % faster per operand
 * so laid out at 2048 x 8192 x 28672.  The three entry points below use it; none has a
 * counterpart in the reference (the recon route, src/torch/amp_torch.cpp:11149-11230, hands
 * row-major tensors to cuBLAS). */

/* exl3_amd_recon_mm with A (a_slabs) and / or WT (w_slabs) in the k-slab layout, and C rows ldc
 * elements apart (ldc >= n, a multiple of 8: C may be a column block of a wider output); results
 * bit for bit those of exl3_amd_recon_mm on the row-major operands. */
int exl3_amd_recon_mm_slabs(const uint16_t* A, const uint16_t* WT, void* C, int c_fp32, const uint16_t* svh,
                            int m, int k, int n, int a_slabs, int w_slabs, int ldc, void* stream);

/* exl3_amd_reconstruct_t (original_basis = 0; suh, svh unused) or exl3_amd_reconstruct_had_t
 * (original_basis = 1) writing WT (n rows of k) in the k-slab layout; k % 32 == 0. */
int exl3_amd_reconstruct_t_slabs(uint16_t* WT, const uint16_t* trellis, const uint16_t* suh,
                                 const uint16_t* svh, int k, int n_packed, int n, int n_offset,
                                 float K, int mcg, int mul1, int original_basis, void* stream);

/* y (rows, cols) in the k-slab layout from x row-major (fp16): a copy (rotate = 0, cols % 32 == 0)
 * or exl3_amd_had_r_128's rotation H128(x o pre) * scale / sqrt(128) (rotate = 1, cols % 128 ==
 * 0).  y must not overlap x. */
int exl3_amd_to_slabs(const uint16_t* x, uint16_t* y, int rows, int cols, int rotate, const uint16_t* pre,
                      float scale, void* stream);

#ifdef __cplusplus
}
#endif
#endif
