// Python module exl3_amd_torch: the at::Tensor operators of exl3_amd_adapter.cpp, called
// exactly as amp_torch.cpp's bindings call them.  c10::Error raised by an operator reaches
// Python as RuntimeError.
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <algorithm>

#include "exl3_amd_adapter.h"

using OptT = c10::optional<at::Tensor>;

PYBIND11_MODULE(exl3_amd_torch, m)
{
    m.def("exl3_gemm", [](const at::Tensor& A, const at::Tensor& B, at::Tensor C, const OptT& suh, const OptT& A_had,
                          const OptT& svh, int force_shape_idx, bool mcg, bool mul1, int force_num_sms) {
        return exl3_gemm(A, B, C, suh, A_had, svh, force_shape_idx, mcg, mul1, force_num_sms);
    });
    m.def("reconstruct", &reconstruct);
    m.def("reconstruct_had_slice", &reconstruct_had_slice);
    m.def("had_r_128", &had_r_128);
    m.def("exl3_mgemm",
          [](const at::Tensor& A, const at::Tensor& B, at::Tensor C, const at::Tensor& suh, const at::Tensor& A_had,
             const at::Tensor& svh, const OptT& indices, const OptT& weights, float K, int force_shape_idx,
             uint32_t mcg_mult, uint32_t mul1_mult, int min_index, int max_index, int force_num_sms, int num_tokens,
             const OptT& size_n_list, const OptT& c_ptrs, const OptT& n_stride_list, const OptT& had_src_list,
             int num_had_src) {
              return exl3_mgemm(A, B, C, suh, A_had, svh, indices, weights, K, force_shape_idx, mcg_mult, mul1_mult,
                                min_index, max_index, force_num_sms, num_tokens, size_n_list, c_ptrs, n_stride_list,
                                had_src_list, num_had_src);
          });
    m.def("exl3_moe_coop",
          [](const at::Tensor& x, const at::Tensor& sel, const at::Tensor& rw, int min_expert, int max_expert, int Hi,
             const at::Tensor& g_trellis, const at::Tensor& g_suh, const at::Tensor& g_svh,
             const at::Tensor& u_trellis, const at::Tensor& u_suh, const at::Tensor& u_svh,
             const at::Tensor& d_trellis, const at::Tensor& d_suh, const at::Tensor& d_svh, const OptT& g_bias,
             const OptT& u_bias, const OptT& d_bias, float Kg, float Ku, float Kd, bool mcg, bool mul1, int act,
             float act_limit, bool gated, at::Tensor had_g, at::Tensor had_u, at::Tensor gu_g, at::Tensor gu_u,
             at::Tensor act_out, at::Tensor d_out, at::Tensor ctr, at::Tensor out, const OptT& sh_out,
             const OptT& sh_gate_w, const OptT& bits_g, const OptT& bits_u, const OptT& bits_d) {
              exl3_moe_coop(x, sel, rw, min_expert, max_expert, Hi, g_trellis, g_suh, g_svh, u_trellis, u_suh, u_svh,
                            d_trellis, d_suh, d_svh, g_bias, u_bias, d_bias, Kg, Ku, Kd, mcg, mul1, act, act_limit,
                            gated, had_g, had_u, gu_g, gu_u, act_out, d_out, ctr, out, sh_out, sh_gate_w, bits_g,
                            bits_u, bits_d);
          });
    m.def("exl3_moe_max_concurrency", &exl3_moe_max_concurrency);
    m.def("exl3_moe_gather", &exl3_moe_gather);
    m.def("exl3_moe", &exl3_moe);
    m.def("rms_norm_res", [](const at::Tensor& x, const at::Tensor& r, const at::Tensor& w, at::Tensor y,
                             at::Tensor n, double eps) {
        const long dim = w.numel();
        const int rc = amp_rms_norm_res_fp16(x.data_ptr(), r.data_ptr(), w.data_ptr(), y.data_ptr(), n.data_ptr(),
                                             x.numel() / std::max(dim, 1L), (int) dim, eps,
                                             (void*) c10::hip::getCurrentHIPStream(x.device().index()).stream());
        TORCH_CHECK(rc == 0, "rms_norm_res: launch failed");
    });
    m.def("silu_mul", [](const at::Tensor& g, const at::Tensor& u, at::Tensor out) {
        const int rc = amp_silu_mul_fp16(g.data_ptr(), u.data_ptr(), out.data_ptr(), g.numel(),
                                         (void*) c10::hip::getCurrentHIPStream(g.device().index()).stream());
        TORCH_CHECK(rc == 0, "silu_mul: launch failed");
    });
}
