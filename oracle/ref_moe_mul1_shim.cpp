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

}
