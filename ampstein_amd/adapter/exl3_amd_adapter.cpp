// at::Tensor front end of libexl3_amd.so: the global C++ operators that ampstein's torch
// bindings declare for the vendored EXL3 kernels (amp_torch.cpp:3739-3896, :11062-11081,
// :7783-7837), with the same signatures.  A ROCm build of amp_torch.cpp drops its
// `#ifndef AMPSTEIN_ROCM` guards around those declarations and links this file and
// libexl3_amd.so instead of the CUDA-only kernel library.
//
// Each operator checks dtypes and ranks the way the vendored TORCH_CHECKs do (the C ABI
// sees only pointers), converts tensors to pointers, launches on the current stream of the
// tensor's device (torch on ROCm reports GPU tensors with device type cuda; the generic
// device guard dispatches to its HIP implementation), and turns a negative C-ABI return code into c10::Error carrying the
// library's message.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <algorithm>
#include <cstdio>

#include "exl3_amd.h"
#include "exl3_amd_adapter.h"

namespace
{

void* cur_stream(const at::Tensor& t)
{
    return (void*) c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

int check(int rc)
{
    TORCH_CHECK(rc >= 0, exl3_amd_last_error());
    return rc;
}

template <class T>
T* opt_ptr(const c10::optional<at::Tensor>& t)
{
    return t.has_value() && t->defined() ? (T*) t->data_ptr() : nullptr;
}

void check_dtype(const at::Tensor& t, at::ScalarType dt, const char* name)
{
    TORCH_CHECK(t.scalar_type() == dt, name, " is incorrect datatype, must be ", c10::toString(dt));
}

void check_on_device(const at::Tensor& t, const char* name)
{
    TORCH_CHECK(t.is_cuda(), name, " must be a GPU tensor");
}

void check_opt(const c10::optional<at::Tensor>& t, at::ScalarType dt, const char* name)
{
    if (t.has_value() && t->defined())
    {
        check_dtype(*t, dt, name);
        check_on_device(*t, name);
    }
}

// trellis tile: 16 K uint16 for integer K, 16 K + 8 for K + 0.5 (bits_k.cuh:8-27)
float K_of_tile(int64_t tile)
{
    return (float) (tile / 16) + (tile % 16 ? 0.5f : 0.0f);
}

}  // namespace

// exl3_gemm.cu:114-350
int exl3_gemm(const at::Tensor& A, const at::Tensor& B, at::Tensor& C,
              const c10::optional<at::Tensor>& suh, const c10::optional<at::Tensor>& A_had,
              const c10::optional<at::Tensor>& svh, int force_shape_idx, bool mcg, bool mul1,
              int force_num_sms)
{
    (void) force_num_sms;       // cooperative-grid override of the CUDA kernel; no meaning here
    TORCH_CHECK(B.dim() == 3, "B must have 3 dimensions");
    TORCH_CHECK(A.dim() >= 1 && A.size(-1) == B.size(0) * 16, "A and B shapes are incompatible");
    TORCH_CHECK(C.dim() >= 1 && C.size(-1) == B.size(1) * 16, "C and B shapes are incompatible");
    check_dtype(A, at::kHalf, "A");
    check_dtype(B, at::kShort, "B");
    const bool c_fp32 = C.scalar_type() == at::kFloat;
    if (!c_fp32) check_dtype(C, at::kHalf, "C");
    TORCH_CHECK(!(mcg && mul1), "Specified both mcg and mul1");
    const int64_t tile = B.size(2);
    TORCH_CHECK(tile % 16 == 0 || (tile % 16 == 8 && mul1),
                "exl3_gemm: half-integer bitrates require the mul1 codebook");
    TORCH_CHECK(A.is_contiguous() && C.is_contiguous() && B.is_contiguous(), "exl3_gemm: tensors must be contiguous");
    check_on_device(A, "A");
    check_on_device(B, "B");
    check_on_device(C, "C");
    check_opt(suh, at::kHalf, "suh");
    check_opt(svh, at::kHalf, "svh");
    check_opt(A_had, at::kHalf, "A_had");
    const int64_t k = A.size(-1);
    const int64_t m = k ? A.numel() / k : 0;
    TORCH_CHECK(C.numel() == m * C.size(-1), "A and C row counts differ");
    if (suh.has_value() && suh->defined()) TORCH_CHECK(suh->numel() >= k, "suh too short");
    if (svh.has_value() && svh->defined()) TORCH_CHECK(svh->numel() >= C.size(-1), "svh too short");
    const c10::OptionalDeviceGuard guard(A.device());
    return check(exl3_amd_gemm((const uint16_t*) A.data_ptr(), (const uint16_t*) B.data_ptr(), C.data_ptr(),
                               c_fp32, opt_ptr<const uint16_t>(suh), opt_ptr<uint16_t>(A_had),
                               opt_ptr<const uint16_t>(svh), (int) m, (int) k, (int) C.size(-1),
                               K_of_tile(tile), mcg, mul1, force_shape_idx, cur_stream(A)));
}

// reconstruct.cu:141-208: n_offset 0, as many columns as `unpacked` holds
void reconstruct(at::Tensor unpacked, at::Tensor packed, float K_, bool mcg, bool mul1)
{
    TORCH_CHECK(unpacked.dim() == 2 && packed.dim() == 3, "reconstruct: bad tensor ranks");
    check_dtype(unpacked, at::kHalf, "unpacked");
    check_dtype(packed, at::kShort, "packed");
    TORCH_CHECK(unpacked.is_contiguous() && packed.is_contiguous(), "reconstruct: tensors must be contiguous");
    if (unpacked.numel() == 0) return;
    check_on_device(unpacked, "unpacked");
    check_on_device(packed, "packed");
    const c10::OptionalDeviceGuard guard(unpacked.device());
    check(exl3_amd_reconstruct((uint16_t*) unpacked.data_ptr(), (const uint16_t*) packed.data_ptr(),
                               (int) unpacked.size(0), (int) packed.size(1) * 16, (int) unpacked.size(1), 0,
                               K_, mcg, mul1, cur_stream(unpacked)));
}

// reconstruct.cu:431-490
void reconstruct_had_slice(at::Tensor unpacked, at::Tensor packed, at::Tensor suh, at::Tensor svh, float K_,
                           bool mcg, bool mul1, int64_t n_offset)
{
    TORCH_CHECK(unpacked.dim() == 2 && packed.dim() == 3, "reconstruct_had: bad tensor ranks");
    check_dtype(unpacked, at::kHalf, "unpacked");
    check_dtype(packed, at::kShort, "packed");
    check_dtype(suh, at::kHalf, "suh");
    check_dtype(svh, at::kHalf, "svh");
    TORCH_CHECK(unpacked.is_contiguous() && packed.is_contiguous(), "reconstruct_had: tensors must be contiguous");
    if (unpacked.numel() == 0) return;
    TORCH_CHECK(suh.numel() >= unpacked.size(0), "reconstruct_had: suh size");
    TORCH_CHECK(svh.numel() >= unpacked.size(1), "reconstruct_had: svh size");
    for (const at::Tensor* t : { &unpacked, &packed, &suh, &svh }) check_on_device(*t, "reconstruct_had operand");
    const c10::OptionalDeviceGuard guard(unpacked.device());
    check(exl3_amd_reconstruct_had((uint16_t*) unpacked.data_ptr(), (const uint16_t*) packed.data_ptr(),
                                   (const uint16_t*) suh.data_ptr(), (const uint16_t*) svh.data_ptr(),
                                   (int) unpacked.size(0), (int) packed.size(1) * 16, (int) unpacked.size(1),
                                   (int) n_offset, K_, mcg, mul1, cur_stream(unpacked)));
}

// hadamard.cu:125-210.  A given pre_scale takes precedence; post_scale is then ignored.
void had_r_128(const at::Tensor& input, const at::Tensor& output, const c10::optional<at::Tensor>& pre_scale,
               const c10::optional<at::Tensor>& post_scale, const float scale)
{
    TORCH_CHECK(input.sizes() == output.sizes(), "input and output shapes differ");
    TORCH_CHECK(input.dim() == 2, "input must have 2 dimensions");
    TORCH_CHECK(input.size(1) % 128 == 0, "input columns must be divisible by 128");
    const bool fp32 = input.scalar_type() == at::kFloat;
    if (fp32) check_dtype(output, at::kFloat, "output");
    else if (input.scalar_type() == at::kHalf) check_dtype(output, at::kHalf, "output");
    else TORCH_CHECK(false, "unsupported datatype");
    TORCH_CHECK(input.is_contiguous() && output.is_contiguous(), "had_r_128: tensors must be contiguous");
    check_opt(pre_scale, at::kHalf, "pre_scale");
    check_opt(post_scale, at::kHalf, "post_scale");
    const uint16_t* pre = opt_ptr<const uint16_t>(pre_scale);
    const uint16_t* post = pre ? nullptr : opt_ptr<const uint16_t>(post_scale);
    if (pre) TORCH_CHECK(pre_scale->numel() >= input.size(1), "scale vector too short");
    if (post) TORCH_CHECK(post_scale->numel() >= input.size(1), "scale vector too short");
    if (input.numel() == 0) return;
    check_on_device(input, "input");
    check_on_device(output, "output");
    const c10::OptionalDeviceGuard guard(input.device());
    check(exl3_amd_had_r_128(input.data_ptr(), output.data_ptr(), (int) input.size(0), (int) input.size(1), fp32,
                             pre, post, scale, cur_stream(input)));
}

// exl3_gemm.cu:396-712 (semantics :352-394).  mcg_mult / mul1_mult select the codebook when
// nonzero, as in the vendored front end (exl3_gemm.cu:696-722).
int exl3_mgemm(const at::Tensor& A, const at::Tensor& B, at::Tensor& C, const at::Tensor& suh,
               const at::Tensor& A_had, const at::Tensor& svh, const c10::optional<at::Tensor>& indices,
               const c10::optional<at::Tensor>& weights, float K, int force_shape_idx, uint32_t mcg_mult,
               uint32_t mul1_mult, int min_index, int max_index, int force_num_sms, int num_tokens,
               const c10::optional<at::Tensor>& size_n_list, const c10::optional<at::Tensor>& c_ptrs,
               const c10::optional<at::Tensor>& n_stride_list, const c10::optional<at::Tensor>& had_src_list,
               int num_had_src)
{
    check_dtype(A, at::kHalf, "A");
    check_dtype(B, at::kLong, "B");
    check_dtype(suh, at::kLong, "suh");
    check_dtype(svh, at::kLong, "svh");
    const bool c_fp32 = C.scalar_type() == at::kFloat;
    if (!c_fp32) check_dtype(C, at::kHalf, "C");
    TORCH_CHECK(A.dim() == 3, "A must have 3 dimensions");
    TORCH_CHECK(B.dim() == 1, "B must have 1 dimension");
    TORCH_CHECK(suh.dim() == 1, "suh must have 1 dimension");
    TORCH_CHECK(svh.dim() == 1, "svh must have 1 dimension");
    TORCH_CHECK(C.dim() == 3, "C must have 3 dimensions");
    TORCH_CHECK(A.size(1) == C.size(1), "A and C shapes are incompatible");
    TORCH_CHECK(A.is_contiguous() && C.is_contiguous(), "exl3_mgemm: A and C must be contiguous");
    for (const at::Tensor* t : { &A, &B, (const at::Tensor*) &C, &suh, &svh }) check_on_device(*t, "exl3_mgemm operand");
    check_opt(indices, at::kLong, "indices");
    check_opt(weights, at::kHalf, "weights");
    check_opt(size_n_list, at::kInt, "size_n_list");
    check_opt(c_ptrs, at::kLong, "c_ptrs");
    check_opt(n_stride_list, at::kInt, "n_stride_list");
    check_opt(had_src_list, at::kInt, "had_src_list");
    const bool has_idx = indices.has_value() && indices->defined();
    if (has_idx) TORCH_CHECK(indices->dim() == 2, "indices must have 2 dimensions");
    if (weights.has_value() && weights->defined()) TORCH_CHECK(weights->dim() == 2, "weights must have 2 dimensions");
    auto count = [](const c10::optional<at::Tensor>& t) { return t.has_value() && t->defined() ? (int) t->size(0) : 0; };
    const bool has_had = A_had.defined() && A_had.numel() > 0;
    if (has_had) check_on_device(A_had, "A_had");
    const c10::OptionalDeviceGuard guard(A.device());
    return check(exl3_amd_mgemm(
        (const uint16_t*) A.data_ptr(), (int) A.size(0), (int) A.size(1), (int) A.size(2),
        (const uint64_t*) B.data_ptr(), (int) B.size(0),
        C.data_ptr(), (int) C.size(0), (int) C.size(2), c_fp32,
        (const uint64_t*) suh.data_ptr(), (int) suh.size(0),
        has_had ? (uint16_t*) A_had.data_ptr() : nullptr, has_had ? A_had.numel() : 0,
        (const uint64_t*) svh.data_ptr(), (int) svh.size(0),
        opt_ptr<const int64_t>(indices), has_idx ? (int) indices->size(1) : 0,
        opt_ptr<const uint16_t>(weights),
        K, force_shape_idx, mcg_mult != 0, mul1_mult != 0, min_index, max_index, force_num_sms, num_tokens,
        opt_ptr<const int>(size_n_list), opt_ptr<const uint64_t>(c_ptrs), count(c_ptrs),
        opt_ptr<const int>(n_stride_list), count(n_stride_list),
        opt_ptr<const int>(had_src_list), count(had_src_list), num_had_src,
        cur_stream(A)));
}

// exl3_moe_coop.cu:307-371, the tensor front end of the fused decode-shaped MoE
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
                   const c10::optional<at::Tensor>& bits_d)
{
    check_dtype(x, at::kHalf, "x");
    check_dtype(sel, at::kLong, "sel");
    check_dtype(rw, at::kHalf, "rw");
    TORCH_CHECK(sel.is_contiguous() && rw.is_contiguous(), "exl3_moe_coop: sel/rw must be contiguous");
    TORCH_CHECK(sel.sizes() == rw.sizes() && sel.dim() == 2 && x.dim() == 2 && sel.size(0) == x.size(0),
                "exl3_moe_coop: sel/rw must be (bsz, topk)");
    TORCH_CHECK(x.stride(1) == 1, "exl3_moe_coop: x must be (bsz, H) with unit column stride");
    check_dtype(ctr, at::kInt, "ctr");
    TORCH_CHECK(ctr.is_contiguous(), "exl3_moe_coop: ctr must be contiguous");
    for (const at::Tensor* t : { &g_trellis, &g_suh, &g_svh, &u_trellis, &u_suh, &u_svh, &d_trellis, &d_suh, &d_svh })
        TORCH_CHECK(t->scalar_type() == at::kLong && t->is_contiguous(),
                    "exl3_moe_coop: pointer tables must be contiguous int64");
    check_dtype(had_g, at::kHalf, "had_g");
    check_dtype(had_u, at::kHalf, "had_u");
    check_dtype(act_out, at::kHalf, "act_out");
    check_dtype(d_out, at::kFloat, "d_out");
    check_dtype(out, at::kFloat, "out");
    TORCH_CHECK((gu_u.scalar_type() == at::kHalf || gu_u.scalar_type() == at::kFloat) &&
                gu_g.scalar_type() == gu_u.scalar_type(), "exl3_moe_coop: gate/up scratch dtype mismatch");
    const int64_t I = gu_u.size(-1), Ho = d_out.size(-1);
    for (auto tw : { std::make_pair(&had_g, (int64_t) Hi), std::make_pair(&had_u, (int64_t) Hi),
                     std::make_pair(&gu_g, I), std::make_pair(&gu_u, I), std::make_pair(&act_out, I),
                     std::make_pair(&d_out, Ho) })
        TORCH_CHECK(tw.first->is_contiguous() && tw.first->size(-1) == tw.second, "exl3_moe_coop: scratch shape");
    TORCH_CHECK(out.dim() >= 2 && out.stride(-1) == 1, "exl3_moe_coop: out shape");
    check_opt(sh_out, at::kFloat, "sh_out");
    if (sh_out.has_value() && sh_out->defined())
        TORCH_CHECK(sh_out->is_contiguous() && sh_out->size(-1) == x.size(1) && sh_out->numel() >= x.numel(),
                    "exl3_moe_coop: shared expert output shape");
    check_opt(sh_gate_w, at::kHalf, "sh_gate_w");
    const int nb = (int) (bits_g.has_value() && bits_g->defined()) + (int) (bits_u.has_value() && bits_u->defined()) +
                   (int) (bits_d.has_value() && bits_d->defined());
    TORCH_CHECK(nb == 0 || nb == 3, "exl3_moe_coop: give all three bit width tables or none");
    for (const c10::optional<at::Tensor>* b : { &bits_g, &bits_u, &bits_d })
        if (b->has_value() && (*b)->defined())
            TORCH_CHECK((*b)->scalar_type() == at::kByte && (*b)->is_contiguous() && (*b)->numel() >= u_trellis.size(0),
                        "exl3_moe_coop: bit width tables must be contiguous uint8, one entry per expert");
    check_opt(g_bias, at::kLong, "g_bias");
    check_opt(u_bias, at::kLong, "u_bias");
    check_opt(d_bias, at::kLong, "d_bias");
    for (const at::Tensor* t : std::initializer_list<const at::Tensor*> { &x, &sel, &rw, &ctr, &out, &had_g, &had_u,
                                                                         &act_out, &d_out, &gu_g, &gu_u })
        check_on_device(*t, "exl3_moe_coop operand");
    const c10::OptionalDeviceGuard guard(x.device());
    check(exl3_amd_moe_coop(
        (const uint16_t*) x.data_ptr(), (int) x.size(0), (int) x.size(1), (int) x.stride(0),
        (const int64_t*) sel.data_ptr(), (const uint16_t*) rw.data_ptr(), (int) sel.size(1),
        min_expert, max_expert, Hi,
        (const uint64_t*) g_trellis.data_ptr(), (const uint64_t*) g_suh.data_ptr(), (const uint64_t*) g_svh.data_ptr(),
        (const uint64_t*) u_trellis.data_ptr(), (const uint64_t*) u_suh.data_ptr(), (const uint64_t*) u_svh.data_ptr(),
        (const uint64_t*) d_trellis.data_ptr(), (const uint64_t*) d_suh.data_ptr(), (const uint64_t*) d_svh.data_ptr(),
        (int) u_trellis.size(0),
        opt_ptr<const uint64_t>(g_bias), opt_ptr<const uint64_t>(u_bias), opt_ptr<const uint64_t>(d_bias),
        Kg, Ku, Kd, mcg, mul1, act, act_limit, gated,
        (uint16_t*) had_g.data_ptr(), had_g.numel(), (uint16_t*) had_u.data_ptr(), had_u.numel(),
        gu_g.data_ptr(), gu_u.data_ptr(), std::min(gu_g.numel(), gu_u.numel()), gu_u.scalar_type() == at::kFloat,
        (int) I, (uint16_t*) act_out.data_ptr(), act_out.numel(),
        (float*) d_out.data_ptr(), d_out.numel(), (int) Ho,
        (int*) ctr.data_ptr(), ctr.numel(),
        (float*) out.data_ptr(), (int) out.size(-2), (int) out.size(-1), (int) out.stride(-2),
        opt_ptr<const float>(sh_out), opt_ptr<const uint16_t>(sh_gate_w),
        sh_gate_w.has_value() && sh_gate_w->defined() ? (int) sh_gate_w->numel() : 0,
        opt_ptr<const uint8_t>(bits_g), opt_ptr<const uint8_t>(bits_u), opt_ptr<const uint8_t>(bits_d),
        cur_stream(x)));
}

int exl3_moe_max_concurrency(int device)
{
    return check(exl3_amd_moe_max_concurrency(device));
}

void exl3_moe_gather(at::Tensor output_state, const at::Tensor& output_scratch, const at::Tensor& flat_expert,
                     const at::Tensor& inv_order, const at::Tensor& expert_start, const at::Tensor& slot_base,
                     const at::Tensor& slot_kind, const at::Tensor& weight_sorted)
{
    // exl3_moe.cu:491-517
    check_dtype(output_state, at::kFloat, "output_state");
    check_dtype(output_scratch, at::kFloat, "output_scratch");
    check_dtype(flat_expert, at::kLong, "flat_expert");
    check_dtype(inv_order, at::kLong, "inv_order");
    check_dtype(expert_start, at::kLong, "expert_start");
    check_dtype(slot_base, at::kLong, "slot_base");
    check_dtype(slot_kind, at::kLong, "slot_kind");
    check_dtype(weight_sorted, at::kHalf, "weight_sorted");
    TORCH_CHECK(output_state.is_contiguous() && output_state.dim() == 2, "exl3_moe_gather: output_state");
    TORCH_CHECK(output_scratch.is_contiguous() && output_scratch.dim() == 2 &&
                output_scratch.size(1) == output_state.size(1), "exl3_moe_gather: output_scratch must be [slots, hidden]");
    TORCH_CHECK(flat_expert.is_contiguous() && inv_order.is_contiguous() && expert_start.is_contiguous() &&
                slot_base.is_contiguous() && slot_kind.is_contiguous() && weight_sorted.is_contiguous(),
                "exl3_moe_gather: index tensors must be contiguous");
    for (const at::Tensor* t : std::initializer_list<const at::Tensor*> { &output_state, &output_scratch, &flat_expert,
                                 &inv_order, &expert_start, &slot_base, &slot_kind, &weight_sorted })
        check_on_device(*t, "exl3_moe_gather operand");
    const c10::OptionalDeviceGuard guard(output_state.device());
    check(exl3_amd_moe_gather((float*) output_state.data_ptr(), (int) output_state.size(0), (int) output_state.size(1),
                              (const float*) output_scratch.data_ptr(), (int) output_scratch.size(1),
                              (const int64_t*) flat_expert.data_ptr(), (int) flat_expert.numel(),
                              (const int64_t*) inv_order.data_ptr(), (const int64_t*) expert_start.data_ptr(),
                              (int) expert_start.numel(), (const int64_t*) slot_base.data_ptr(), (int) slot_base.numel(),
                              (const int64_t*) slot_kind.data_ptr(), (int) slot_kind.numel(),
                              (const uint16_t*) weight_sorted.data_ptr(), cur_stream(output_state)));
}

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
              const c10::optional<at::Tensor>& bits_d)
{
    // exl3_moe.cu:186-235: tensor checks; the rest are made by the C ABI in the same order
    if (num_active == 0) return;
    const bool scr = output_scratch.has_value() && output_scratch->defined();
    if (scr)
    {
        TORCH_CHECK(fused_base.has_value() && fused_base->defined(), "exl3_moe: output_scratch needs fused_base");
        check_dtype(*output_scratch, at::kFloat, "output_scratch");
        check_dtype(*fused_base, at::kLong, "fused_base");
        TORCH_CHECK(output_scratch->is_contiguous() && output_scratch->dim() == 2 &&
                    output_scratch->size(1) == hidden_state.size(1), "exl3_moe: output_scratch must be [slots, hidden]");
    }
    check_dtype(hidden_state, at::kHalf, "hidden_state");
    TORCH_CHECK(hidden_state.dim() == 2 && hidden_state.is_contiguous(), "hidden_state must be 2-dimensional");
    check_dtype(output_state, at::kFloat, "output_state");
    TORCH_CHECK(output_state.sizes() == hidden_state.sizes(), "output_state and hidden_state shapes differ");
    check_dtype(expert_count, at::kLong, "expert_count");
    TORCH_CHECK(expert_count.dim() == 1, "expert_count must be 1-dimensional");
    check_dtype(token_sorted, at::kLong, "token_sorted");
    TORCH_CHECK(token_sorted.dim() == 1 && token_sorted.sizes() == weight_sorted.sizes(),
                "token_sorted and weight_sorted shapes differ");
    check_dtype(weight_sorted, at::kHalf, "weight_sorted");
    for (const at::Tensor* t : { &temp_state_g, &temp_state_u, &temp_intermediate_g, &temp_intermediate_u })
    {
        check_dtype(*t, at::kHalf, "temp buffer");
        TORCH_CHECK(t->dim() == 3 && t->is_contiguous(), "exl3_moe: temp buffers must be contiguous and 3-dimensional");
    }
    TORCH_CHECK(temp_state_g.size(2) == hidden_state.size(1) && temp_state_g.sizes() == temp_state_u.sizes(),
                "temp_state shapes differ");
    TORCH_CHECK(temp_intermediate_g.sizes() == temp_intermediate_u.sizes() &&
                temp_intermediate_g.size(1) == temp_state_g.size(1), "temp_intermediate shapes differ");
    for (const at::Tensor* t : { &gate_ptrs_trellis, &gate_ptrs_suh, &gate_ptrs_svh, &up_ptrs_trellis, &up_ptrs_suh,
                                 &up_ptrs_svh, &down_ptrs_trellis, &down_ptrs_suh, &down_ptrs_svh })
        TORCH_CHECK(t->scalar_type() == at::kLong && t->dim() == 1 && t->is_contiguous() &&
                    t->sizes() == gate_ptrs_trellis.sizes(), "exl3_moe: pointer tables must be contiguous int64 of one length");
    const int nb = (int) (bits_g.has_value() && bits_g->defined()) + (int) (bits_u.has_value() && bits_u->defined()) +
                   (int) (bits_d.has_value() && bits_d->defined());
    TORCH_CHECK(nb == 0 || nb == 3, "exl3_moe: give all three bit width tables or none");
    for (const c10::optional<at::Tensor>* b : { &bits_g, &bits_u, &bits_d })
        if (b->has_value() && (*b)->defined())
            TORCH_CHECK((*b)->scalar_type() == at::kByte && (*b)->is_contiguous() && (*b)->numel() >= expert_count.numel() - 1,
                        "exl3_moe: bit width tables must be contiguous uint8, one entry per expert");
    for (const at::Tensor* t : { &hidden_state, &output_state, &expert_count, &token_sorted, &weight_sorted,
                                 &temp_state_g, &temp_intermediate_g })
        check_on_device(*t, "exl3_moe operand");
    const c10::OptionalDeviceGuard guard(hidden_state.device());
    check(exl3_amd_moe(
        (const uint16_t*) hidden_state.data_ptr(), (int) hidden_state.size(0), (int) hidden_state.size(1),
        (float*) output_state.data_ptr(), (const int64_t*) expert_count.data_ptr(), (int) expert_count.numel(),
        (const int64_t*) token_sorted.data_ptr(), (const uint16_t*) weight_sorted.data_ptr(), (int) token_sorted.numel(),
        (uint16_t*) temp_state_g.data_ptr(), (uint16_t*) temp_state_u.data_ptr(), (int) temp_state_g.size(0),
        (int) temp_state_g.size(1), (uint16_t*) temp_intermediate_g.data_ptr(), (uint16_t*) temp_intermediate_u.data_ptr(),
        (int) temp_intermediate_g.size(2), act_function, K_gate, K_up, K_down,
        (const uint64_t*) gate_ptrs_trellis.data_ptr(), (const uint64_t*) gate_ptrs_suh.data_ptr(),
        (const uint64_t*) gate_ptrs_svh.data_ptr(), (const uint64_t*) up_ptrs_trellis.data_ptr(),
        (const uint64_t*) up_ptrs_suh.data_ptr(), (const uint64_t*) up_ptrs_svh.data_ptr(),
        (const uint64_t*) down_ptrs_trellis.data_ptr(), (const uint64_t*) down_ptrs_suh.data_ptr(),
        (const uint64_t*) down_ptrs_svh.data_ptr(), (int) gate_ptrs_trellis.numel(),
        gate_mcg, gate_mul1, up_mcg, up_mul1, down_mcg, down_mul1, act_limit, num_active,
        scr ? (float*) output_scratch->data_ptr() : nullptr, scr ? output_scratch->size(0) : 0,
        scr ? (int) output_scratch->size(1) : 0, scr ? (const int64_t*) fused_base->data_ptr() : nullptr,
        count_lo, count_hi, m_tile, opt_ptr<const uint8_t>(bits_g), opt_ptr<const uint8_t>(bits_u),
        opt_ptr<const uint8_t>(bits_d), nb ? (int) bits_g->numel() : 0, cur_stream(hidden_state)));
}

// amp_kernels.cu:253-268 / :367-397 return a HIP status (0 = launched); a rejected argument
// prints the library's message, as the reference prints its dim check, and returns -1.
extern "C" int amp_silu_mul_fp16(const void* g, const void* u, void* out, long n, void* stream)
{
    const int rc = exl3_amd_silu_mul((const uint16_t*) g, (const uint16_t*) u, (uint16_t*) out, n, stream);
    if (rc < 0) fprintf(stderr, "amp_silu_mul: %s\n", exl3_amd_last_error());
    return rc < 0 ? -1 : 0;
}

extern "C" int amp_rms_norm_res_fp16(const void* x, const void* r, const void* w, void* y, void* n, long rows,
                                     int dim, double eps, void* stream)
{
    const int rc = exl3_amd_rms_norm_res((const uint16_t*) x, (const uint16_t*) r, (const uint16_t*) w,
                                         (uint16_t*) y, (uint16_t*) n, rows, dim, (float) eps, stream);
    if (rc < 0) fprintf(stderr, "amp_rms_norm_res: %s\n", exl3_amd_last_error());
    return rc < 0 ? -1 : 0;
}
