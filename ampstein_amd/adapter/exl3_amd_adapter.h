// Declarations of the EXL3 operators that ampstein's torch bindings call, with the
// signatures of amp_torch.cpp:3739-3896 (exl3_moe_coop, exl3_gemm, reconstruct,
// exl3_mgemm) and :11062-11081 (had_r_128, reconstruct_had_slice).  Defined over
// libexl3_amd.so in exl3_amd_adapter.cpp.
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
