// Declarations of the EXL3 operators that ampstein's torch bindings call, with the
// signatures of amp_torch.cpp:3739-3896 (exl3_moe_coop, exl3_gemm, reconstruct,
// exl3_mgemm), :7783-7837 (exl3_moe_max_concurrency, exl3_moe_gather, exl3_moe),
// :11062-11081 (had_r_128, reconstruct_had_slice) and the two decode-step kernels of
// :4433-4439 (amp_silu_mul_fp16, amp_rms_norm_res_fp16).  Defined over libexl3_amd.so in
// exl3_amd_adapter.cpp.
#pragma once

#include <ATen/ATen.h>
#include <c10/util/Optional.h>

#include <cstdint>

void exl3_moe_coop(const at::Tensor& x, const at::Tensor& sel, const at::Tensor& rw, int min_expert,
                   int max_expert, int Hi,
                   const at::Tensor& g_trellis, const at::Tensor& g_suh, const at::Tensor& g_svh,
                   const at::Tensor& u_trellis, const at::Tensor& u_suh, const at::Tensor& u_svh,
                   const at::Tensor& d_trellis, const at::Tensor& d_suh, const at::Tensor& d_svh,
                   const c10::optional<at::Tensor>& g_bias, const c10::optional<at::Tensor>& u_bias,
                   const c10::optional<at::Tensor>& d_bias, float Kg, float Ku, float Kd, bool mcg, bool mul1,
                   int act, float act_limit, bool gated, at::Tensor& had_g, at::Tensor& had_u, at::Tensor& gu_g,
                   at::Tensor& gu_u, at::Tensor& act_out, at::Tensor& d_out, at::Tensor& ctr, at::Tensor& out,
                   const c10::optional<at::Tensor>& sh_out, const c10::optional<at::Tensor>& sh_gate_w,
                   const c10::optional<at::Tensor>& bits_g, const c10::optional<at::Tensor>& bits_u,
                   const c10::optional<at::Tensor>& bits_d);

int exl3_gemm(const at::Tensor& A, const at::Tensor& B, at::Tensor& C,
              const c10::optional<at::Tensor>& suh, const c10::optional<at::Tensor>& A_had,
              const c10::optional<at::Tensor>& svh, int force_shape_idx, bool mcg, bool mul1,
              int force_num_sms);

void reconstruct(at::Tensor unpacked, at::Tensor packed, float K_, bool mcg, bool mul1);

int exl3_mgemm(const at::Tensor& A, const at::Tensor& B, at::Tensor& C, const at::Tensor& suh,
               const at::Tensor& A_had, const at::Tensor& svh, const c10::optional<at::Tensor>& indices,
               const c10::optional<at::Tensor>& weights, float K, int force_shape_idx, uint32_t mcg_mult,
               uint32_t mul1_mult, int min_index, int max_index, int force_num_sms, int num_tokens = 1,
               const c10::optional<at::Tensor>& size_n_list = {}, const c10::optional<at::Tensor>& c_ptrs = {},
               const c10::optional<at::Tensor>& n_stride_list = {},
               const c10::optional<at::Tensor>& had_src_list = {}, int num_had_src = 0);

void had_r_128(const at::Tensor& input, const at::Tensor& output, const c10::optional<at::Tensor>& pre_scale,
               const c10::optional<at::Tensor>& post_scale, const float scale);

void reconstruct_had_slice(at::Tensor unpacked, at::Tensor packed, at::Tensor suh, at::Tensor svh, float K_,
                           bool mcg, bool mul1, int64_t n_offset);

int exl3_moe_max_concurrency(int device);

void exl3_moe_gather(at::Tensor output_state, const at::Tensor& output_scratch, const at::Tensor& flat_expert,
                     const at::Tensor& inv_order, const at::Tensor& expert_start, const at::Tensor& slot_base,
                     const at::Tensor& slot_kind, const at::Tensor& weight_sorted);

void exl3_moe(const at::Tensor& hidden_state, const at::Tensor& output_state, const at::Tensor& expert_count,
              const at::Tensor& token_sorted, const at::Tensor& weight_sorted, const at::Tensor& temp_state_g,
              const at::Tensor& temp_state_u, const at::Tensor& temp_intermediate_g,
              const at::Tensor& temp_intermediate_u, const int act_function, const float K_gate, const float K_up,
              const float K_down, const at::Tensor& gate_ptrs_trellis, const at::Tensor& gate_ptrs_suh,
              const at::Tensor& gate_ptrs_svh, const at::Tensor& up_ptrs_trellis, const at::Tensor& up_ptrs_suh,
              const at::Tensor& up_ptrs_svh, const at::Tensor& down_ptrs_trellis, const at::Tensor& down_ptrs_suh,
              const at::Tensor& down_ptrs_svh, const bool gate_mcg, const bool gate_mul1, const bool up_mcg,
              const bool up_mul1, const bool down_mcg, const bool down_mul1, const float act_limit,
              const int num_active, const c10::optional<at::Tensor>& output_scratch,
              const c10::optional<at::Tensor>& fused_base, const int count_lo, const int count_hi, const int m_tile,
              const c10::optional<at::Tensor>& bits_g, const c10::optional<at::Tensor>& bits_u,
              const c10::optional<at::Tensor>& bits_d);

// The decode-step kernels the bindings call with raw pointers (the stream is a hipStream_t).
extern "C" int amp_silu_mul_fp16(const void* g, const void* u, void* out, long n, void* stream);
extern "C" int amp_rms_norm_res_fp16(const void* x, const void* r, const void* w, void* y, void* n, long rows,
                                     int dim, double eps, void* stream);
