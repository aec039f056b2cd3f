// Build shim for oracle/_ref: compiles the reference's own CPU expert kernel source
// (vendor/exl3/exllamav3_ext/cpu/moe_mul1.cpp, included from /root/reference where it lies)
// and exposes its scalar format helpers through a C ABI so the tests can check the oracle's
// restatement against them. TEST INFRASTRUCTURE ONLY; nothing here ships.
#include REF_MOE_MUL1_CPP

extern "C" {

// moe_mul1.cpp:125-139
void ref_tc_perm(uint16_t* out)
{
    const auto p = make_tc_perm();
    for (int i = 0; i < 256; ++i) out[i] = p[i];
}

// moe_mul1.cpp:190-200 (integer K only in the reference)
int ref_decode_state(int bits, const uint16_t* packed, int t)
{
    switch (bits)
    {
        case 1: return decode_state_scalar<1>(packed, t);
        case 2: return decode_state_scalar<2>(packed, t);
        case 3: return decode_state_scalar<3>(packed, t);
        case 4: return decode_state_scalar<4>(packed, t);
        case 5: return decode_state_scalar<5>(packed, t);
        case 6: return decode_state_scalar<6>(packed, t);
        case 7: return decode_state_scalar<7>(packed, t);
        case 8: return decode_state_scalar<8>(packed, t);
    }
    return -1;
}

// moe_mul1.cpp:78-83: window end of ring position t (HALF25 = the 2.5 bpw ring)
int ref_window_end(int bits, int t)
{
    switch (bits)
    {
        case 1: return window_end<1>(t);
        case 2: return window_end<2>(t);
        case 3: return window_end<3>(t);
        case 4: return window_end<4>(t);
        case 5: return window_end<5>(t);
        case 6: return window_end<6>(t);
        case 7: return window_end<7>(t);
        case 8: return window_end<8>(t);
        case 25: return window_end<HALF25>(t);
    }
    return -1;
}

// moe_mul1.cpp:223-237
void ref_hadamard_128_scalar(float* v) { hadamard_128_scalar(v); }

// moe_mul1.cpp:202-207 (fp32 form of the mul1 value)
float ref_decode_mul1_scalar(uint16_t s) { return decode_mul1_scalar(s); }


// moe_mul1.cpp:2418-2474 (exl3_moe_cpu_make_layer) and :2529-2654 (exl3_moe_cpu_forward_raw):
// the reference's CPU MoE forward on E mul1 experts.  mats[3 * e + p] for p = gate, up, down
// (gate entries ignored when !gated); biases may be NULL.  Returns 0, or -1 when the reference
// rejects the arguments.
int ref_moe_forward(int E, int H, int I, const int* bits, int gated,
                    const uint16_t* const* trellis, const uint16_t* const* suh,
                    const uint16_t* const* svh, const uint16_t* const* bias,
                    int activation, float limit, const uint16_t* x, const int* sel,
                    const uint16_t* w, float* out, int rows, int topk)
{
    try
    {
        auto i16 = torch::TensorOptions().dtype(torch::kInt16);
        auto f16 = torch::TensorOptions().dtype(torch::kHalf);
        std::vector<at::Tensor> tr[3], su[3], sv[3], bi[3];
        for (int e = 0; e < E; ++e)
            for (int p = 0; p < 3; ++p)
            {
                if (p == 0 && !gated) continue;
                const int k = p == 2 ? I : H, n = p == 2 ? H : I;
                const int q = 3 * e + p;
                tr[p].push_back(torch::from_blob((void*) trellis[q], {k / 16, n / 16, 16 * bits[e]}, i16));
                su[p].push_back(torch::from_blob((void*) suh[q], {k}, f16));
                sv[p].push_back(torch::from_blob((void*) svh[q], {n}, f16));
                if (bias) bi[p].push_back(torch::from_blob((void*) bias[q], {n}, f16));
            }
        int64_t hd = exl3_moe_cpu_make_layer(tr[0], su[0], sv[0], tr[1], su[1], sv[1], tr[2], su[2],
                                             sv[2], bi[0], bi[1], bi[2], activation, limit, 0);
        exl3_moe_cpu_forward_raw(hd, (const at::Half*) x, sel, (const at::Half*) w, out, rows, topk, 1);
        exl3_moe_cpu_free_layer(hd);
        return 0;
    }
    catch (const std::exception&)
    {
        return -1;
    }
}

}
