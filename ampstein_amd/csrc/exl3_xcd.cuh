// Device side of the per-launch XCD hand-off check (XcdGuard, exl3_kernels.h).
//
// The last arrival at a hand-off counter reads the other arrivals' split-k partials through its
// own XCD's L2; partials stored on another XCD stay in that XCD's L2 (the workgroup-scope release
// writes nothing back).  The counter therefore records who arrived: it is one 64-bit word, and
// every arrival adds 1 + (v << 16) + (v^2 << 32) with v = XCC id + 1, so that the last arrival
// holds n = count, S1 = sum of v and S2 = sum of v^2.  n S2 = S1^2 exactly when every v is equal
// (equality case of Cauchy-Schwarz); otherwise the launch's sums cannot be trusted and the last
// arrival stores 1 to the host-visible alarm word.  Atomic read-modify-writes are performed at a
// point coherent across XCDs (device-wide atomics rely on it), so the count is exact either way.
// No memory operation is added to the hand-off: the check rides on the counter's own atomic.
// Fields: count < 2^16, S1 < 2^16, S2 < 2^32 for up to 3000 arrivals of v <= 18.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "exl3_common.cuh"
#include "exl3_kernels.h"

namespace exl3 {

// The increment of this workgroup's arrival (uniform: XCC id from the hardware register).
__device__ __forceinline__ uint64_t xcd_increment(const XcdGuard& q)
{
    uint32_t x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(x));
    const int lin = (int) (blockIdx.x + blockIdx.y * gridDim.x);
    const uint64_t v = x + 1u + (lin == q.fake_block ? 1u : 0u);
    return 1ull | (v << 16) | ((v * v) << 32);
}

// Count one arrival; true for the last of `total`.  The last arrival checks the XCC record and
// re-arms the counter (64-bit zero).
__device__ __forceinline__ bool xcd_arrive(const XcdGuard& q, int* ctr, int total)
{
    uint64_t* c = (uint64_t*) ctr;
    const uint64_t inc = xcd_increment(q);
    const uint64_t prev = __hip_atomic_fetch_add(to_global_w(c), inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const uint64_t cur = prev + inc;
    const uint32_t n = (uint32_t) (cur & 0xffffu);
    if ((int) n != total) return false;
    const uint64_t s1 = (cur >> 16) & 0xffffu, s2 = cur >> 32;
    if ((uint64_t) n * s2 != s1 * s1) __hip_atomic_store(q.alarm, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(to_global_w(c), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return true;
}

}  // namespace exl3
