// C-ABI entry points of libexl3_amd.so (declared in include/exl3_amd.h).
//
// Every argument check of the reference's TORCH_CHECKs for these operators is made here,
// before any launch, and reported as an error code plus a thread-local message instead of
// an exception (quant/reconstruct.cu:152-176, hadamard.cu:141-145, exl3_gemm.cu:128-176,
// bits_k.cuh:178-185).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <atomic>
#include <mutex>
#include <string>

#include "../../include/exl3_amd.h"
#include "exl3_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int hip_fail(int rc, const char* what)
{
    if (rc == -1) return fail(EXL3_AMD_EUNSUPPORTED, "%s: no kernel instance for this bitrate/codebook", what);
    return fail(EXL3_AMD_EHIP, "%s: HIP error %d (%s)", what, rc, hipGetErrorString((hipError_t) rc));
}

// Bitrate K: integer 1..8, or 1.5 / 2.5 / 3.5 with the mul1 codebook (bits_k.cuh:178-185).
// *bits receives the rate code: the integer bitrate, or 16 + b for b + 1/2.
// both_ok: the reconstruct entry points take mcg over mul1 when both are set
// (reconstruct.cu:181-184); exl3_gemm rejects the combination (exl3_gemm.cu:179).
int parse_K(float K, int mcg, int mul1, int* bits, int* half, int* cb, const char* what, bool both_ok = false)
{
    const int b = (int) K;
    const float f = K - (float) b;
    if (!(b >= 1 && b <= 8 && (f == 0.0f || (f == 0.5f && b <= 3))))
        return fail(EXL3_AMD_EINVAL, "%s: unsupported EXL3 bitrate %g (integer 1..8, or 1.5 / 2.5 / 3.5)", what, (double) K);
    if (mcg && mul1 && !both_ok) return fail(EXL3_AMD_EINVAL, "%s: specified both mcg and mul1", what);
    *half = f == 0.5f;
    *bits = *half ? 16 + b : b;         // the kernels' rate code (exl3_common.cuh kbits / khalf)
    *cb = mcg ? 1 : (mul1 ? 2 : 0);
    if (*half && mul1) *cb = 2;
    if (*half && !mul1) return fail(EXL3_AMD_EINVAL, "%s: half-integer bitrates require the mul1 codebook", what);
    return 0;
}

// ------------------------------------------------------------------ per-device workspace
constexpr int MAX_DEVICES = 16;
constexpr size_t WS_PARTIAL_BYTES = 64ull << 20;     // split-k fp32 partials
constexpr size_t WS_COUNTERS = 1u << 20;             // column-chunk completion counters
// the fused norm's row counter: its own 128-byte line after every other counter range
constexpr size_t WS_NORM_CTR = WS_COUNTERS;
constexpr size_t WS_COUNTER_INTS = WS_COUNTERS + 32;

struct DeviceState
{
    bool ready = false;
    int num_cus = 0;
    int num_xcd = 0;            // > 0 when workgroup b is verified to run on XCD b % num_xcd
    int probe_xcd = 0;          // the init probe's verdict (num_xcd until the hand-off check trips)
    int xcd_alarms = 0;         // alarms serviced (the hand-off check saw one counter on two XCDs)
    uint32_t* alarm_host = nullptr;     // pinned, device-mapped alarm word (host view)
    uint32_t* alarm_dev = nullptr;      // the same word's device address
    float* partials = nullptr;
    int* counters = nullptr;
    uint32_t* sink = nullptr;           // 8 KiB, zeroed, never written after init
    int64_t* filt_idx = nullptr;      // mgemm expert-range filter output (MGEMM_MAX_FILTER slots)
    uint16_t* filt_w = nullptr;
};
constexpr int MGEMM_MAX_FILTER = 128;   // exl3_gemm_kernel.cuh:82 (index-compaction capacity)

DeviceState g_dev[MAX_DEVICES];
std::mutex g_mutex;

// Kernel-path policy (exl3_amd_set_policy): the library's defaults unless a test or benchmark
// selects an alternative path explicitly.  Read once per call.
std::atomic<int> g_policy[EXL3_AMD_POLICY_COUNT];

int policy(int key) { return g_policy[key].load(std::memory_order_relaxed); }

// ------------------------------------------------------------------ allocation-free scratch
// exl3_amd_gemm_noalloc's device memory: one file-scope array, present on every GPU the library
// runs on until the process ends.  Layout: split-k partials | completion counters | prefetch sink.
// The counters and the sink start at zero (static initialisation); every kernel that counts
// re-arms its counter before it ends, and nothing writes the sink, so both are zero again after
// each call.  Calls on one GPU share the array: calls that overlap on one GPU race.
constexpr size_t NOALLOC_PARTIAL_BYTES = 16u << 20;
constexpr size_t NOALLOC_COUNTER_INTS = 64u << 10;
constexpr size_t NOALLOC_SINK_BYTES = 8192;
constexpr size_t NOALLOC_SCRATCH_BYTES = NOALLOC_PARTIAL_BYTES + NOALLOC_COUNTER_INTS * sizeof(int) + NOALLOC_SINK_BYTES;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

struct NoAllocState
{
    bool ready = false;
    unsigned char* ptr = nullptr;       // this device's copy of scratch (hipGetSymbolAddress)
    int num_cus = 0;
};
NoAllocState g_noalloc[MAX_DEVICES];

// Once per device, with that device current: the device address of its scratch copy.  The
// array's name in host code is only a host-side handle; kernels receive this address.
int noalloc_setup(int device)
{
    if (device < 0 || device >= MAX_DEVICES) return fail(EXL3_AMD_EINVAL, "device %d out of range", device);
    NoAllocState& st = g_noalloc[device];
    if (st.ready) return 0;
    std::lock_guard<std::mutex> lock(g_mutex);
    if (st.ready) return 0;
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
    {
        (void) hipGetLastError();
        return fail(EXL3_AMD_EHIP, "scratch symbol address on device %d: HIP error %d (%s)", device, (int) e,
                    hipGetErrorString(e));
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
        return fail(EXL3_AMD_EHIP, "device attribute query failed");
    st.ptr = (unsigned char*) ptr;
    st.num_cus = cus;
    st.ready = true;
    return 0;
}

int init_device(int device, DeviceState** out)
{
    if (device < 0 || device >= MAX_DEVICES) return fail(EXL3_AMD_EINVAL, "device %d out of range", device);
    DeviceState& d = g_dev[device];
    if (!d.ready)
    {
        std::lock_guard<std::mutex> lock(g_mutex);
        if (!d.ready)
        {
            int prev = 0;
            hipGetDevice(&prev);
            if (prev != device && hipSetDevice(device) != hipSuccess)
                return fail(EXL3_AMD_EHIP, "hipSetDevice(%d) failed", device);
            int cus = 0;
            if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
                return fail(EXL3_AMD_EHIP, "device attribute query failed");
            void* p = nullptr;
            void* c = nullptr;
            if (hipMalloc(&p, WS_PARTIAL_BYTES) != hipSuccess) return fail(EXL3_AMD_ENOMEM, "workspace allocation failed");
            if (hipMalloc(&c, WS_COUNTER_INTS * sizeof(int)) != hipSuccess)
            {
                (void) hipFree(p);
                return fail(EXL3_AMD_ENOMEM, "counter allocation failed");
            }
            if (hipMemset(c, 0, WS_COUNTER_INTS * sizeof(int)) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
                return fail(EXL3_AMD_EHIP, "counter initialisation failed");
            void* f = nullptr;
            if (hipMalloc(&f, MGEMM_MAX_FILTER * (sizeof(int64_t) + sizeof(uint16_t))) != hipSuccess)
                return fail(EXL3_AMD_ENOMEM, "filter workspace allocation failed");
            void* sk = nullptr;
            if (hipMalloc(&sk, 8192) != hipSuccess) return fail(EXL3_AMD_ENOMEM, "sink allocation failed");
            if (hipMemset(sk, 0, 8192) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
                return fail(EXL3_AMD_EHIP, "sink initialisation failed");
            d.sink = (uint32_t*) sk;
            // hand-off check: the alarm word (pinned host memory that kernels store to with system
            // scope, read by the host at every call)
            // (without it the hand-off stays off: every launch must be checkable)
            void* al = nullptr;
            void* al_dev = nullptr;
            if (hipHostMalloc(&al, 64, hipHostMallocMapped | hipHostMallocCoherent) == hipSuccess && al)
            {
                memset(al, 0, 64);
                if (hipHostGetDevicePointer(&al_dev, al, 0) == hipSuccess && al_dev)
                {
                    d.alarm_host = (uint32_t*) al;
                    d.alarm_dev = (uint32_t*) al_dev;
                }
            }
            (void) hipGetLastError();
            d.filt_idx = (int64_t*) f;
            d.filt_w = (uint16_t*) (d.filt_idx + MGEMM_MAX_FILTER);
            // workgroup -> XCD dispatch order (round-robin on MI355X), verified on this device
            {
                const int gx[4] = { 64, 1000, 8192, 64 }, gy[4] = { 1, 1, 1, 9 };
                int* probe = (int*) p;
                int nx = 0;
                bool ok = true;
                // the probe's launch status is read with hipGetLastError: drop any error an earlier
                // call of the host process (not this library) left pending
                (void) hipGetLastError();
                for (int si = 0; si < 4 && ok; ++si)
                {
                    const int total = gx[si] * gy[si];
                    int* host = (int*) malloc(total * sizeof(int));
                    if (!host || exl3k_xcd_probe(probe, gx[si], gy[si], nullptr) || hipDeviceSynchronize() != hipSuccess ||
                        hipMemcpy(host, probe, total * sizeof(int), hipMemcpyDeviceToHost) != hipSuccess)
                        ok = false;
                    if (ok)
                    {
                        int mx = 0;
                        for (int i = 0; i < total; ++i) mx = host[i] > mx ? host[i] : mx;
                        if (si == 0) nx = mx + 1;
                        // linear workgroup id (x fastest) -> XCD, round-robin from wherever the
                        // previous dispatch on the queue left off: workgroups b and b + nx share an
                        // XCD, which is all the hand-off needs
                        for (int i = 0; i < total && ok; ++i) ok = host[i] == (host[0] + i) % nx;
                    }
                    if (getenv("EXL3_AMD_DEBUG") && host)
                        fprintf(stderr, "exl3_amd: xcd probe %d (%dx%d): ok %d nx %d first %d %d %d %d %d %d %d %d %d\n", si,
                                gx[si], gy[si], (int) ok, nx, host[0], host[1], host[2], host[3], host[4], host[5], host[6],
                                host[7], host[8]);
                    free(host);
                }
                d.num_xcd = ok && nx >= 1 && nx <= 31 && d.alarm_dev ? nx : 0;
                if (const char* e = getenv("EXL3_AMD_XCD")) if (atoi(e) == 0) d.num_xcd = 0;
                d.probe_xcd = d.num_xcd;
            }
            d.num_cus = cus;
            d.partials = (float*) p;
            d.counters = (int*) c;
            d.ready = true;
            if (prev != device) (void) hipSetDevice(prev);
        }
    }
    *out = &d;
    return 0;
}

// Every entry point that launches comes through here.  The launchers report their launch
// status with hipGetLastError, so a stale error left by other code in the process is dropped
// first: it would otherwise be reported as this call's failure.
// The first call on a device allocates and clears the workspace, which a stream capture cannot
// record: such a call is refused (no allocation, no synchronisation) and the capture stays
// intact.  exl3_amd_init(device) before the capture avoids it.
// Makes `device` current for the scope (calls that take a device argument and
// synchronise, copy or launch on it).
struct DeviceScope
{
    int prev = -1;
    explicit DeviceScope(int device)
    {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != device) (void) hipSetDevice(device);
    }
    ~DeviceScope() { if (prev >= 0) (void) hipSetDevice(prev); }
};

// The XCD hand-off check's alarm (set by a kernel that saw one counter's arrivals come from two
// XCDs): turn the hand-off off for the device and zero every counter on `s`, so
// that no later call reads what the mixed launch left.  Called by every entry point that launches
// work; a plain host read of pinned memory when nothing happened.
void xcd_service(int device, hipStream_t s)
{
    DeviceState& d = g_dev[device];
    if (!d.ready || !d.alarm_host || d.num_xcd == 0) return;
    if (__atomic_load_n(d.alarm_host, __ATOMIC_ACQUIRE) == 0) return;
    std::lock_guard<std::mutex> lock(g_mutex);
    if (d.num_xcd == 0) return;
    d.num_xcd = 0;
    ++d.xcd_alarms;
    fprintf(stderr, "exl3_amd: device %d: workgroups of one split-k hand-off counter ran on different XCDs; the "
            "XCD-local hand-off is now off for this device (outputs of the launch that raised this are not reliable)\n",
            device);
    (void) exl3k_fill_u32((uint32_t*) d.counters, 0u, WS_COUNTER_INTS, s);
    const NoAllocState& st = g_noalloc[device];
    if (st.ready)
    {
        (void) exl3k_fill_u32((uint32_t*) (st.ptr + NOALLOC_PARTIAL_BYTES), 0u, NOALLOC_COUNTER_INTS, s);
    }
}

// The guard the kernels of one launch carry.
XcdGuard xcd_guard(uint32_t* alarm)
{
    const int fake = policy(EXL3_AMD_POLICY_XCD_FAKE);
    return XcdGuard { alarm, fake > 0 ? fake - 1 : -1 };
}

// Most arrivals one 64-bit hand-off counter records (16-bit count and id-sum fields).
constexpr int XCD_MAX_ARRIVALS = 3000;

int current_device(DeviceState** out, void* stream)
{
    (void) hipGetLastError();
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(EXL3_AMD_EHIP, "hipGetDevice failed");
    if (dev >= 0 && dev < MAX_DEVICES && !g_dev[dev].ready)
    {
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing((hipStream_t) stream, &st) != hipSuccess || st != hipStreamCaptureStatusNone)
        {
            (void) hipGetLastError();
            return fail(EXL3_AMD_EINVAL, "first call on device %d during stream capture: the workspace is allocated "
                        "on first use; call exl3_amd_init(%d) before capturing", dev, dev);
        }
    }
    if (int rc = init_device(dev, out)) return rc;
    xcd_service(dev, (hipStream_t) stream);
    return 0;
}

// Row-batched matrix-core GEMV (exl3_gemv.hip gemvm_kernel) for 2..16 rows (policy
// EXL3_AMD_POLICY_GEMV_ROWS: 0 = default; EXL3_AMD_GEMV_ROWS_LDS keeps the LDS kernel for up to
// 8 rows, EXL3_AMD_GEMV_ROWS_MFMA_ALL also takes single rows there).  Returns 0 (LDS kernel),
// 1 (matrix cores from 2 rows) or 2 (matrix cores from 1 row).
int gemv_mfma_mode()
{
    switch (policy(EXL3_AMD_POLICY_GEMV_ROWS))
    {
        case EXL3_AMD_GEMV_ROWS_LDS: return 0;
        case EXL3_AMD_GEMV_ROWS_MFMA_ALL: return 2;
    }
    return 1;
}

// Work-split constants of the GEMV planner (measured on MI355X; see the comments at their uses).
constexpr int GEMVM_TARGET_WG_PER_CU_X2 = 3;     // matrix-core GEMV: 1.5 workgroups per CU
constexpr int GEMVM_STAGED_X_BYTES = 48 * 1024;  // its staged input rows, per workgroup
constexpr int GEMV_LDS_WG_PER_CU = 4;            // LDS / stream kernels: 4 workgroups per CU

// GEMV work split (exl3_gemv.hip): SB slices per workgroup, a divisor of k/16 (so no
// workgroup straddles two column chunks), sized for ~TARGET workgroups per CU within the LDS
// budget (rotated input + reduction buffer) and the split-partial workspace.
int gemv_plan(int m, int k, int n, int bszm, int num_cus, GemvArgs& g, size_t partial_bytes = WS_PARTIAL_BYTES)
{
    {
        const int mode = gemv_mfma_mode();
        const bool use = m <= 16 && (m >= 2 ? mode != 0 : mode >= 2);
        if (use)
        {
            const int KS = k / 16, chunks = n / 128;
            const int mt = m == 1 ? 1 : (m <= 4 ? 4 : (m <= 8 ? 8 : 16));
            // target grid: 1.5 workgroups per CU
            const long target = (long) GEMVM_TARGET_WG_PER_CU_X2 * num_cus / 2;
            // SB: k-tiles per workgroup, a multiple of 8 dividing k/16, at most 64 (16 units per
            // wave; 32 for 16 rows); the largest whose grid still reaches the target (else the smallest), within
            // 48 KB of staged input and the workspace.  Measured on MI355X over SB (Qwen 5120 x
            // {5120, 17408}, 17408 x 5120, m = 1..16): the optimum sits at 1.5-2.7 workgroups per
            // CU with SB 32-64; SB 8 (the most workgroups) is up to 1.5x slower.
            int best = -1;
            const int sb_max = mt >= 16 ? 32 : 64;                // 16 rows: SB 32 measured best
            for (int d = 8; d <= KS && d <= sb_max; d += 8)
            {
                if (KS % d) continue;
                if ((size_t) mt * (d * 16 + 4) * 4 > (size_t) GEMVM_STAGED_X_BYTES) break;
                if ((size_t) (KS / d) * bszm * m * n * 4 > partial_bytes && KS / d > 1) continue;
                if ((long) bszm * chunks * (KS / d) >= target || best < 0) best = d;
                if ((long) bszm * chunks * (KS / d) < target) break;
            }
            if (best > 0)
            {
                g.stream_m1 = 0;
                g.mfma_rows = 1;
                g.slices_per_block = best;
                g.slots = KS / best;
                g.xs_chunks = 0;
                return 0;
            }
        }
    }
    // the LDS and stream kernels hold at most 8 rows: a group of 9..16 rows whose matrix-core
    // plan did not fit is split by the caller (launch_gemv)
    if (m > 8) return -1;
    g.mfma_rows = 0;
    const int mt = m == 1 ? 1 : (m <= 4 ? 4 : 8);
    const int KS = k / 16, chunks = n / 128;
    const long target = (long) GEMV_LDS_WG_PER_CU * num_cus;
    // M = 1 streaming kernel: 1, 2 or 4 slices per wave, or whole 128-row input chunks (SB % 32 == 0)
    const int stream = m == 1;
    auto ok_sb = [&](int d) { return KS % d == 0 && (!stream || d == 4 || d == 8 || d == 16 || d % 32 == 0); };
    const int lds_budget = 64 * 1024 - 4 * mt * 128 * 4;
    const int max_chunks = lds_budget / (mt * 512);           // rotated 128-row chunks in LDS
    int best = -1;
    for (int d = stream ? 4 : 1; d <= KS; ++d)
    {
        if (!ok_sb(d)) continue;
        if (!stream && d / 8 + 2 > max_chunks) break;
        if ((size_t) (KS / d) * bszm * m * n * 4 > partial_bytes && KS / d > 1) continue;
        if (best < 0 || (long) bszm * chunks * (KS / best) > target) best = d;   // fewest blocks >= target
        if ((long) bszm * chunks * (KS / d) <= target) break;
    }
    // M = 1 stream: 4 k-slices per wave below k = 8192, 16 from there: the best splits measured
    // on MI355X for the Llama-3-8B shapes in a captured sweep (4096 x 4096: 6.85 -> 6.45 us, the
    // sliced q/k/v bundle 9.1 -> 7.9 us against 8 per wave; 14336 x 4096 best at 16)
    if (stream)
    {
        int pref = k >= 8192 ? 64 : 16;
        // more than 8 workgroups per CU: double the split while the count exceeds that (measured
        // with the 2-slice prefetch ring, 32-layer graph sweep, us per launch at 16 / 32 / 64 / 128
        // slices per workgroup: stacked gate / up 23.3 / 21.6 / 22.3 / 23.4 -> 32, 1792 workgroups)
        while (ok_sb(2 * pref) && (long) bszm * chunks * (KS / pref) > 8L * num_cus) pref *= 2;
        for (int d = pref; d >= 4; d /= 2)
            if (ok_sb(d) && ((size_t) (KS / d) * bszm * m * n * 4 <= partial_bytes || KS / d == 1)) { best = d; break; }
        // policy EXL3_AMD_POLICY_GEMV_SLICES: a forced split (k-slices per workgroup) when valid
        const int forced = policy(EXL3_AMD_POLICY_GEMV_SLICES);
        if (forced > 0 && ok_sb(forced) && ((size_t) (KS / forced) * bszm * m * n * 4 <= partial_bytes || KS / forced == 1))
            best = forced;
    }
    if (best < 0) return -1;
    if ((size_t) (KS / best) * bszm * m * n * 4 > partial_bytes && KS / best > 1) return -1;
    g.stream_m1 = stream;
    g.slices_per_block = best;
    g.slots = KS / best;
    g.xs_chunks = best / 8 + 2;
    return 0;
}

GemvArgs gemv_args_single(const uint16_t* A, const uint16_t* trellis, void* C, int c_fp32,
                          const uint16_t* suh, const uint16_t* svh, int m, int k, int n)
{
    GemvArgs g;
    memset(&g, 0, sizeof(g));
    g.A = A; g.trellis = trellis; g.C = C; g.suh = suh; g.svh = svh;
    g.m = m; g.k = k; g.n = n; g.c_fp32 = c_fp32 ? 1 : 0;
    g.bszm_in = 1; g.bszm = 1; g.num_tokens = 1;
    return g;
}

int dispatch_gemv(int bits, int cb, const GemvArgs& g, hipStream_t s);

#ifdef EXL3_GEMV_TRACE
uint64_t* g_trace = nullptr;
#endif

// Device memory the GEMV kernels use beyond inputs and outputs: split-k partials, completion
// counters (zero between calls: every kernel that counts re-arms its counter), the prefetch sink.
struct Workspace
{
    float* partials;
    size_t partial_bytes;
    int* counters;
    size_t counter_ints;
    const uint32_t* sink;
    int num_cus;
    int num_xcd;
    uint32_t* alarm;            // device address of the alarm word
};

Workspace ws_of(const DeviceState* d)
{
    return Workspace { d->partials, WS_PARTIAL_BYTES, d->counters, WS_COUNTERS, d->sink, d->num_cus, d->num_xcd,
                       d->alarm_dev };
}

// Balanced M = 1 stream (exl3_gemv.hip gemv1b_kernel): every wave streams the same R slices of
// the residue-ordered pair list and every SIMD holds the same number of waves (4, else 3 or 2),
// R >= 4 and 4 R <= k/16 (a workgroup's range meets two pairs at most).  Plain single-row
// launches only (no routing weights, indices, per-matrix widths, fused input or norm), integer
// 3INST / MCG, XCD hand-off on.
void plan_balanced(GemvArgs& g, const Workspace& w, int bits)
{
    if (g.A_up || g.norm_h || g.res_h || g.in_w || g.weights || g.indices || g.size_n || g.had_src || g.c_list || g.row0 || bits > 8)
        return;
    const long KS = g.k / 16, P = (long) g.bszm * (g.n / 128);
    if (P % g.xcd) return;
    for (int wps = 4; wps >= 2; --wps)
    {
        const long waves = (long) wps * 4 * w.num_cus;
        if ((P * KS) % waves) continue;
        const long R = P * KS / waves;
        if (R < 4 || 4 * R > KS || waves % (4L * g.xcd)) continue;
        const long S = (KS + 4 * R - 1) / (4 * R) + 1;     // most workgroups one pair can meet
        if ((size_t) P * S * 128 * 4 > w.partial_bytes) continue;
        g.stream_m1 = 2;
        g.slices_per_block = (int) R;
        g.slots = (int) S;
        return;
    }
}

// Plan the work split, pick the XCD hand-off when the device and shape allow it, launch.
int launch_gemv(const Workspace& w, int bits, int cb, GemvArgs& g, hipStream_t s, const char* what)
{
    const int chunks = g.n / 128;
    if (gemv_plan(g.m, g.k, g.n, g.bszm, w.num_cus, g, w.partial_bytes))
    {
        // a 9..16-row group whose matrix-core plan exceeds the split-partial workspace (or with
        // the matrix-core GEMV off): two launches of at most 8 rows, rows [row0, row0 + 8) and
        // the rest, on the same slabs
        if (g.m > 8)
        {
            GemvArgs lo = g, hi = g;
            if (!g.slab_m) lo.slab_m = hi.slab_m = g.m;
            lo.m = 8;
            hi.m = g.m - 8;
            hi.row0 = g.row0 + 8;
            if (int rc = launch_gemv(w, bits, cb, lo, s, what)) return rc;
            return launch_gemv(w, bits, cb, hi, s, what);
        }
        return fail(EXL3_AMD_EUNSUPPORTED, "%s: shape exceeds the GEMV workspace (%zu bytes of split partials)", what,
                    w.partial_bytes);
    }
    g.partials = w.partials;
    g.counters = w.counters;
    g.counters_half = (int) (w.counter_ints / 2);
    g.sink = w.sink;
#ifdef EXL3_GEMV_TRACE
    g.trace = g_trace;
#endif
    const size_t pairs = (size_t) g.bszm * chunks;
    g.xcd = 0;
    if (w.num_xcd > 0 && w.alarm && chunks % w.num_xcd == 0 && pairs * 32 <= w.counter_ints / 2 &&
        g.slots <= XCD_MAX_ARRIVALS && g.bszm <= XCD_MAX_ARRIVALS)
        g.xcd = w.num_xcd;
    g.xg = xcd_guard(w.alarm);
    if (g.xcd && g.m == 1 && g.stream_m1 == 1 && cb != 2 && policy(EXL3_AMD_POLICY_GEMV_SPLIT) == EXL3_AMD_GEMV_SPLIT_BALANCED)
        plan_balanced(g, w, bits);
    if (g.in_w && !(g.m == 1 && g.stream_m1 == 1 && g.k <= 64 * SQ_SCALE_MAX_PER_LANE * 128))
    {
        // the other kernels read a formed input: the split norm's consumer half as its own launch
        const int rows = g.slab_m ? g.slab_m : g.m;
        if (int rc = exl3k_norm_sq(g.A, g.in_sq, g.in_w, g.in_r, rows, g.k, g.in_eps, s)) return hip_fail(rc, what);
        g.A = g.in_r;
        g.in_w = nullptr;
        g.in_sq = nullptr;
    }
    int rc = dispatch_gemv(bits, cb, g, s);
    return rc ? hip_fail(rc, what) : 0;
}

int dispatch_gemm(int bits, int cb, const GemmArgs& g, hipStream_t s)
{
    switch (bits)
    {
        case 1: return exl3k_gemm_k1(g, cb, s);
        case 2: return exl3k_gemm_k2(g, cb, s);
        case 3: return exl3k_gemm_k3(g, cb, s);
        case 4: return exl3k_gemm_k4(g, cb, s);
        case 5: return exl3k_gemm_k5(g, cb, s);
        case 6: return exl3k_gemm_k6(g, cb, s);
        case 7: return exl3k_gemm_k7(g, cb, s);
        case 8: return exl3k_gemm_k8(g, cb, s);
        case 17: return exl3k_gemm_k17(g, cb, s);
        case 18: return exl3k_gemm_k18(g, cb, s);
        case 19: return exl3k_gemm_k19(g, cb, s);
    }
    return -1;
}

int dispatch_gemv(int bits, int cb, const GemvArgs& g, hipStream_t s)
{
    switch (bits)
    {
        case 1: return exl3k_gemv_k1(g, cb, s);
        case 2: return exl3k_gemv_k2(g, cb, s);
        case 3: return exl3k_gemv_k3(g, cb, s);
        case 4: return exl3k_gemv_k4(g, cb, s);
        case 5: return exl3k_gemv_k5(g, cb, s);
        case 6: return exl3k_gemv_k6(g, cb, s);
        case 7: return exl3k_gemv_k7(g, cb, s);
        case 8: return exl3k_gemv_k8(g, cb, s);
        case 17: return exl3k_gemv_k17(g, cb, s);
        case 18: return exl3k_gemv_k18(g, cb, s);
        case 19: return exl3k_gemv_k19(g, cb, s);
    }
    return -1;
}

}  // namespace

extern "C" {

#ifdef EXL3_GEMV_TRACE
void exl3_amd_debug_set_trace(void* p) { g_trace = (uint64_t*) p; }
#endif

const char* exl3_amd_last_error(void) { return g_last_error.c_str(); }

int exl3_amd_version(void) { return 10200; }

int exl3_amd_set_policy(int key, int value)
{
    g_last_error.clear();
    if (key < 0 || key >= EXL3_AMD_POLICY_COUNT) return fail(EXL3_AMD_EINVAL, "set_policy: unknown key %d", key);
    g_policy[key].store(value, std::memory_order_relaxed);
    return 0;
}

int exl3_amd_get_policy(int key)
{
    if (key < 0 || key >= EXL3_AMD_POLICY_COUNT) return fail(EXL3_AMD_EINVAL, "get_policy: unknown key %d", key);
    return policy(key);
}

int exl3_amd_init(int device)
{
    DeviceState* d;
    if (int rc = init_device(device, &d)) return rc;
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess) return fail(EXL3_AMD_EHIP, "hipGetDevice failed");
    if (prev != device && hipSetDevice(device) != hipSuccess) return fail(EXL3_AMD_EHIP, "hipSetDevice(%d) failed", device);
    const int rc = noalloc_setup(device);
    if (prev != device) (void) hipSetDevice(prev);
    return rc;
}

int exl3_amd_debug_read_workspace(int device, int64_t offset, int64_t bytes, void* host_dst)
{
    g_last_error.clear();
    DeviceState* d;
    if (int rc = init_device(device, &d)) return rc;
    if (offset < 0 || bytes < 0 || (uint64_t) (offset + bytes) > WS_PARTIAL_BYTES || (bytes && !host_dst))
        return fail(EXL3_AMD_EINVAL, "debug_read_workspace: range outside the %zu-byte workspace", WS_PARTIAL_BYTES);
    DeviceScope scope(device);
    if (hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(host_dst, (char*) d->partials + offset, (size_t) bytes, hipMemcpyDeviceToHost) != hipSuccess)
        return fail(EXL3_AMD_EHIP, "debug_read_workspace: copy failed");
    return 0;
}

int exl3_amd_debug_fill_workspace(int device, int byte_value)
{
    g_last_error.clear();
    DeviceState* d;
    if (int rc = init_device(device, &d)) return rc;
    DeviceScope scope(device);
    if (hipDeviceSynchronize() != hipSuccess || hipMemset(d->partials, byte_value & 0xff, WS_PARTIAL_BYTES) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess)
        return fail(EXL3_AMD_EHIP, "debug_fill_workspace: memset failed");
    return 0;
}

int exl3_amd_device_info(int device, int* num_cus, int* num_xcd)
{
    DeviceState* d;
    if (int rc = init_device(device, &d)) return rc;
    if (num_cus) *num_cus = d->num_cus;
    if (num_xcd) *num_xcd = d->num_xcd;
    return 0;
}

int exl3_amd_xcd_status(int device, int* probe_xcd, int* active_xcd, int* alarms)
{
    g_last_error.clear();
    DeviceState* d;
    if (int rc = init_device(device, &d)) return rc;
    DeviceScope scope(device);
    if (hipDeviceSynchronize() != hipSuccess) return fail(EXL3_AMD_EHIP, "xcd_status: device synchronisation failed");
    xcd_service(device, nullptr);
    if (hipDeviceSynchronize() != hipSuccess) return fail(EXL3_AMD_EHIP, "xcd_status: device synchronisation failed");
    if (probe_xcd) *probe_xcd = d->probe_xcd;
    if (active_xcd) *active_xcd = d->num_xcd;
    if (alarms) *alarms = d->xcd_alarms;
    return 0;
}

int exl3_amd_xcd_rearm(int device)
{
    g_last_error.clear();
    DeviceState* d;
    if (int rc = init_device(device, &d)) return rc;
    DeviceScope scope(device);
    std::lock_guard<std::mutex> lock(g_mutex);
    if (hipDeviceSynchronize() != hipSuccess ||
        hipMemset(d->counters, 0, WS_COUNTER_INTS * sizeof(int)) != hipSuccess)
        return fail(EXL3_AMD_EHIP, "xcd_rearm: reset failed");
    const NoAllocState& st = g_noalloc[device];
    if (st.ready && hipMemset(st.ptr + NOALLOC_PARTIAL_BYTES, 0, NOALLOC_COUNTER_INTS * sizeof(int)) != hipSuccess)
        return fail(EXL3_AMD_EHIP, "xcd_rearm: reset failed");
    if (hipDeviceSynchronize() != hipSuccess) return fail(EXL3_AMD_EHIP, "xcd_rearm: reset failed");
    __atomic_store_n(d->alarm_host, 0u, __ATOMIC_RELEASE);
    d->num_xcd = d->probe_xcd;
    return 0;
}

int exl3_amd_debug_handoff_map(int kind, int xcd, int p0, int p1, int p2, int b, int* out)
{
    g_last_error.clear();
    if (!out || b < 0) return fail(EXL3_AMD_EINVAL, "debug_handoff_map: bad argument");
    switch (kind)
    {
    case 0:
        if (p0 < 1) return fail(EXL3_AMD_EINVAL, "debug_handoff_map: splits must be positive");
        gemv_block_coords(xcd, p0, b, out[0], out[1]);
        return 0;
    case 1:
        if (p0 < 1 || (xcd > 0 && p0 % xcd)) return fail(EXL3_AMD_EINVAL, "debug_handoff_map: bad chunk count");
        moe_chunk_coords(xcd, p0, b, out[0], out[1]);
        return 0;
    case 2:
    {
        // plan_balanced's invariants: whole workgroups of 4 R slices per residue list, 4 R <= k / 16
        if (xcd < 1 || p0 < 1 || p0 % xcd || p1 < 1 || p2 < 1 || 4 * p2 > p1 || ((long) p0 / xcd * p1) % (4L * p2))
            return fail(EXL3_AMD_EINVAL, "debug_handoff_map: bad balanced plan");
        Gemv1bBlock o { 0, 0, 0, false };
        const bool v = gemv1b_block(xcd, p0, p1, p2, b, o);
        out[0] = v; out[1] = o.pa; out[2] = o.pb; out[3] = o.straddle;
        return 0;
    }
    case 3:
        if (p1 < 1 || p2 < 1) return fail(EXL3_AMD_EINVAL, "debug_handoff_map: bad balanced plan");
        gemv1b_pair_span(p1, p2, b, out[0], out[1]);
        return 0;
    default:
        return fail(EXL3_AMD_EINVAL, "debug_handoff_map: unknown kind %d", kind);
    }
}

int exl3_amd_reconstruct(uint16_t* W, const uint16_t* trellis, int k, int n_packed, int n,
                         int n_offset, float K, int mcg, int mul1, void* stream)
{
    g_last_error.clear();
    int bits, half, cb;
    if (int rc = parse_K(K, mcg, mul1, &bits, &half, &cb, "reconstruct", true)) return rc;
    if (k < 0 || n < 0 || n_packed < 0) return fail(EXL3_AMD_EINVAL, "reconstruct: negative size");
    if (k % 16 || n_packed % 16) return fail(EXL3_AMD_EINVAL, "reconstruct: k and the packed width must be multiples of 16");
    if ((size_t) k * n == 0) return 0;
    if (!W || !trellis) return fail(EXL3_AMD_EINVAL, "reconstruct: null pointer");
    if (n % 128) return fail(EXL3_AMD_EINVAL, "unpacked N dimension must be divisible by 128");
    if (n_offset % 128) return fail(EXL3_AMD_EINVAL, "n_offset must be divisible by 128");
    if (n_offset < 0) return fail(EXL3_AMD_EINVAL, "n_offset must be non-negative");
    if (n_offset + n > n_packed) return fail(EXL3_AMD_EINVAL, "reconstruct slice exceeds packed tensor bounds");
    int rc = exl3k_reconstruct(W, trellis, k, n, n_packed / 16, n_offset / 16, bits, cb, (hipStream_t) stream);
    return rc ? hip_fail(rc, "reconstruct") : 0;
}

static int reconstruct_t_impl(uint16_t* WT, const uint16_t* trellis, int k, int n_packed, int n,
                              int n_offset, float K, int mcg, int mul1, int slabs, void* stream)
{
    int bits, half, cb;
    if (int rc = parse_K(K, mcg, mul1, &bits, &half, &cb, "reconstruct_t", true)) return rc;
    if (k < 0 || n < 0 || n_packed < 0) return fail(EXL3_AMD_EINVAL, "reconstruct_t: negative size");
    if (slabs && k % 32) return fail(EXL3_AMD_EINVAL, "reconstruct_t: k must be a multiple of 32 for the slab layout");
    if (k % 16 || n_packed % 16) return fail(EXL3_AMD_EINVAL, "reconstruct_t: k and the packed width must be multiples of 16");
    if ((size_t) k * n == 0) return 0;
    if (!WT || !trellis) return fail(EXL3_AMD_EINVAL, "reconstruct_t: null pointer");
    if (n % 128) return fail(EXL3_AMD_EINVAL, "reconstruct_t: N dimension must be divisible by 128");
    if (n_offset % 128 || n_offset < 0) return fail(EXL3_AMD_EINVAL, "reconstruct_t: n_offset must be a non-negative multiple of 128");
    if (n_offset + n > n_packed) return fail(EXL3_AMD_EINVAL, "reconstruct slice exceeds packed tensor bounds");
    DeviceState* d;
    if (int rc = current_device(&d, stream)) return rc;
    int rc = exl3k_reconstruct_tr(WT, trellis, k, n, n_packed / 16, n_offset / 16, bits, cb, nullptr, slabs,
                                  (hipStream_t) stream);
    return rc ? hip_fail(rc, "reconstruct_t") : 0;
}

int exl3_amd_reconstruct_t(uint16_t* WT, const uint16_t* trellis, int k, int n_packed, int n,
                           int n_offset, float K, int mcg, int mul1, void* stream)
{
    g_last_error.clear();
    return reconstruct_t_impl(WT, trellis, k, n_packed, n, n_offset, K, mcg, mul1, 0, stream);
}

int exl3_amd_reconstruct_t_had(uint16_t* WT, const uint16_t* trellis, const uint16_t* svh, int k, int n_packed,
                               int n, int n_offset, float K, int mcg, int mul1, void* stream)
{
    g_last_error.clear();
    int bits, half, cb;
    if (int rc = parse_K(K, mcg, mul1, &bits, &half, &cb, "reconstruct_t_had", true)) return rc;
    if (k < 0 || n < 0 || n_packed < 0) return fail(EXL3_AMD_EINVAL, "reconstruct_t_had: negative size");
    if (k % 16 || n_packed % 16) return fail(EXL3_AMD_EINVAL, "reconstruct_t_had: k and the packed width must be multiples of 16");
    if ((size_t) k * n == 0) return 0;
    if (!WT || !trellis || !svh) return fail(EXL3_AMD_EINVAL, "reconstruct_t_had: null pointer");
    if (n % 128) return fail(EXL3_AMD_EINVAL, "reconstruct_t_had: N dimension must be divisible by 128");
    if (n_offset % 128 || n_offset < 0) return fail(EXL3_AMD_EINVAL, "reconstruct_t_had: n_offset must be a non-negative multiple of 128");
    if (n_offset + n > n_packed) return fail(EXL3_AMD_EINVAL, "reconstruct slice exceeds packed tensor bounds");
    DeviceState* d;
    if (int rc = current_device(&d, stream)) return rc;
    int rc = exl3k_reconstruct_tr(WT, trellis, k, n, n_packed / 16, n_offset / 16, bits, cb, svh + n_offset, 0,
                                  (hipStream_t) stream);
    return rc ? hip_fail(rc, "reconstruct_t_had") : 0;
}

int exl3_amd_reconstruct_had(uint16_t* W, const uint16_t* trellis, const uint16_t* suh,
                             const uint16_t* svh, int k, int n_packed, int n, int n_offset,
                             float K, int mcg, int mul1, void* stream)
{
    g_last_error.clear();
    int bits, half, cb;
    if (int rc = parse_K(K, mcg, mul1, &bits, &half, &cb, "reconstruct_had", true)) return rc;
    if (k < 0 || n < 0 || n_packed < 0) return fail(EXL3_AMD_EINVAL, "reconstruct_had: negative size");
    if ((size_t) k * n == 0) return 0;
    if (!W || !trellis || !suh || !svh) return fail(EXL3_AMD_EINVAL, "reconstruct_had: null pointer");
    if (k % 128) return fail(EXL3_AMD_EINVAL, "reconstruct_had: K dimension must be divisible by 128");
    if (n % 128) return fail(EXL3_AMD_EINVAL, "reconstruct_had: N dimension must be divisible by 128");
    if (n_packed % 16) return fail(EXL3_AMD_EINVAL, "reconstruct_had: packed width must be a multiple of 16");
    if (n_offset % 128) return fail(EXL3_AMD_EINVAL, "n_offset must be divisible by 128");
    if (n_offset < 0) return fail(EXL3_AMD_EINVAL, "n_offset must be non-negative");
    if (n_offset + n > n_packed) return fail(EXL3_AMD_EINVAL, "reconstruct slice exceeds packed tensor bounds");
    int rc = exl3k_reconstruct_had(W, trellis, suh, svh, k, n, n_packed / 16, n_offset / 16, bits, cb,
                                   (hipStream_t) stream);
    return rc ? hip_fail(rc, "reconstruct_had") : 0;
}

static int reconstruct_had_t_impl(uint16_t* WT, const uint16_t* trellis, const uint16_t* suh,
                                  const uint16_t* svh, int k, int n_packed, int n, int n_offset,
                                  float K, int mcg, int mul1, int slabs, void* stream)
{
    int bits, half, cb;
    if (int rc = parse_K(K, mcg, mul1, &bits, &half, &cb, "reconstruct_had_t", true)) return rc;
    if (k < 0 || n < 0 || n_packed < 0) return fail(EXL3_AMD_EINVAL, "reconstruct_had_t: negative size");
    if ((size_t) k * n == 0) return 0;
    if (!WT || !trellis || !suh || !svh) return fail(EXL3_AMD_EINVAL, "reconstruct_had_t: null pointer");
    if (k % 128) return fail(EXL3_AMD_EINVAL, "reconstruct_had_t: K dimension must be divisible by 128");
    if (n % 128) return fail(EXL3_AMD_EINVAL, "reconstruct_had_t: N dimension must be divisible by 128");
    if (n_packed % 16) return fail(EXL3_AMD_EINVAL, "reconstruct_had_t: packed width must be a multiple of 16");
    if (n_offset % 128) return fail(EXL3_AMD_EINVAL, "n_offset must be divisible by 128");
    if (n_offset < 0) return fail(EXL3_AMD_EINVAL, "n_offset must be non-negative");
    if (n_offset + n > n_packed) return fail(EXL3_AMD_EINVAL, "reconstruct slice exceeds packed tensor bounds");
    int rc = exl3k_reconstruct_had_tr(WT, trellis, suh, svh, k, n, n_packed / 16, n_offset / 16, bits, cb, slabs,
                                      (hipStream_t) stream);
    return rc ? hip_fail(rc, "reconstruct_had_t") : 0;
}

int exl3_amd_reconstruct_had_t(uint16_t* WT, const uint16_t* trellis, const uint16_t* suh,
                               const uint16_t* svh, int k, int n_packed, int n, int n_offset,
                               float K, int mcg, int mul1, void* stream)
{
    g_last_error.clear();
    return reconstruct_had_t_impl(WT, trellis, suh, svh, k, n_packed, n, n_offset, K, mcg, mul1, 0, stream);
}

int exl3_amd_reconstruct_t_slabs(uint16_t* WT, const uint16_t* trellis, const uint16_t* suh,
                                 const uint16_t* svh, int k, int n_packed, int n, int n_offset,
                                 float K, int mcg, int mul1, int original_basis, void* stream)
{
    g_last_error.clear();
    if (original_basis)
        return reconstruct_had_t_impl(WT, trellis, suh, svh, k, n_packed, n, n_offset, K, mcg, mul1, 1, stream);
    return reconstruct_t_impl(WT, trellis, k, n_packed, n, n_offset, K, mcg, mul1, 1, stream);
}

static int recon_mm_impl(const uint16_t* A, const uint16_t* WT, void* C, int c_fp32, const uint16_t* svh,
                         int m, int k, int n, int a_slabs, int w_slabs, int ldc, void* stream)
{
    if (m < 0 || k < 0 || n < 0) return fail(EXL3_AMD_EINVAL, "recon_mm: negative size");
    if (k % 32) return fail(EXL3_AMD_EINVAL, "recon_mm: k must be a multiple of 32");
    if (n % 128) return fail(EXL3_AMD_EINVAL, "recon_mm: n must be a multiple of 128");
    if ((size_t) m * n == 0) return 0;
    if (k == 0) return fail(EXL3_AMD_EINVAL, "recon_mm: k must be positive");
    if (!A || !WT || !C) return fail(EXL3_AMD_EINVAL, "recon_mm: null pointer");
    if (ldc < n || ldc % 8) return fail(EXL3_AMD_EINVAL, "recon_mm: output row stride must be >= n and a multiple of 8");
    // the library workspace holds the split-k partial tiles
    DeviceState* d;
    if (int rc = current_device(&d, stream)) return rc;
    int rc = exl3k_dense_gemm(A, WT, C, c_fp32 ? 1 : 0, svh, m, k, n, a_slabs ? 1 : 0, w_slabs ? 1 : 0, ldc,
                              policy(EXL3_AMD_POLICY_RECON_MM), d->num_cus, d->partials, WS_PARTIAL_BYTES,
                              (hipStream_t) stream);
    return rc ? hip_fail(rc, "recon_mm") : 0;
}

int exl3_amd_recon_mm(const uint16_t* A, const uint16_t* WT, void* C, int c_fp32, const uint16_t* svh,
                      int m, int k, int n, void* stream)
{
    g_last_error.clear();
    return recon_mm_impl(A, WT, C, c_fp32, svh, m, k, n, 0, 0, n, stream);
}

int exl3_amd_recon_mm_slabs(const uint16_t* A, const uint16_t* WT, void* C, int c_fp32, const uint16_t* svh,
                            int m, int k, int n, int a_slabs, int w_slabs, int ldc, void* stream)
{
    g_last_error.clear();
    return recon_mm_impl(A, WT, C, c_fp32, svh, m, k, n, a_slabs, w_slabs, ldc, stream);
}

int exl3_amd_had_r_128(const void* x, void* y, int rows, int cols, int fp32,
                       const uint16_t* pre, const uint16_t* post, float scale, void* stream)
{
    g_last_error.clear();
    if (rows < 0 || cols < 0) return fail(EXL3_AMD_EINVAL, "had_r_128: negative size");
    if (cols % 128) return fail(EXL3_AMD_EINVAL, "had_r_128: columns must be divisible by 128");
    if (pre && post) return fail(EXL3_AMD_EINVAL, "had_r_128: give pre or post scale, not both");
    if ((size_t) rows * cols == 0) return 0;
    if (!x || !y) return fail(EXL3_AMD_EINVAL, "had_r_128: null pointer");
    int rc = exl3k_had128(x, y, rows, cols, fp32 ? 1 : 0, pre, post, scale, 0, (hipStream_t) stream);
    return rc ? hip_fail(rc, "had_r_128") : 0;
}

int exl3_amd_to_slabs(const uint16_t* x, uint16_t* y, int rows, int cols, int rotate, const uint16_t* pre,
                      float scale, void* stream)
{
    g_last_error.clear();
    if (rows < 0 || cols < 0) return fail(EXL3_AMD_EINVAL, "to_slabs: negative size");
    if (cols % (rotate ? 128 : 32)) return fail(EXL3_AMD_EINVAL, "to_slabs: columns must be divisible by %d", rotate ? 128 : 32);
    if ((size_t) rows * cols == 0) return 0;
    if (!x || !y) return fail(EXL3_AMD_EINVAL, "to_slabs: null pointer");
    if (x == y) return fail(EXL3_AMD_EINVAL, "to_slabs: the output cannot overwrite the input");
    if (!rotate && pre) return fail(EXL3_AMD_EINVAL, "to_slabs: a pre scale needs the rotation");
    (void) hipGetLastError();
    int rc = rotate ? exl3k_had128(x, y, rows, cols, 0, pre, nullptr, scale, 1, (hipStream_t) stream)
                    : exl3k_slab_copy(x, y, rows, cols, (hipStream_t) stream);
    return rc ? hip_fail(rc, "to_slabs") : 0;
}

}  // extern "C"

namespace {

// exl3_gemm on a given workspace (the library's per-device one, or the no-alloc scratch).
// ws == nullptr: the library's, set up on first use.
int gemm_impl(const Workspace* ws, const uint16_t* A, const uint16_t* trellis, void* C, int c_fp32,
              const uint16_t* suh, uint16_t* A_had, const uint16_t* svh,
              int m, int k, int n, float K, int mcg, int mul1, int force_shape_idx,
              void* stream, const char* name)
{
    g_last_error.clear();
    int bits, half, cb;
    if (int rc = parse_K(K, mcg, mul1, &bits, &half, &cb, name)) return rc;
    if (m < 0 || k < 0 || n < 0) return fail(EXL3_AMD_EINVAL, "%s: negative size", name);
    if (k % 16) return fail(EXL3_AMD_EINVAL, "%s: k must be a multiple of 16", name);
    if (n % 128) return fail(EXL3_AMD_EINVAL, "%s: n must be a multiple of 128", name);
    if (m == 0 || n == 0) return EXL3_AMD_TAG_GEMV;
    if (!A || !trellis || !C) return fail(EXL3_AMD_EINVAL, "%s: null pointer", name);
    if (k == 0) return fail(EXL3_AMD_EINVAL, "%s: k must be positive", name);
    if (k % 128) return fail(EXL3_AMD_EUNSUPPORTED, "%s: k %% 128 != 0 is not implemented in this build", name);
    if (force_shape_idx > 2) return fail(EXL3_AMD_EINVAL, "%s: bad force_shape_idx %d", name, force_shape_idx);

    Workspace lw;
    if (!ws)
    {
        DeviceState* d;
        if (int rc = current_device(&d, stream)) return rc;
        lw = ws_of(d);
        ws = &lw;
    }
    else (void) hipGetLastError();
    hipStream_t s = (hipStream_t) stream;

    if (m <= 8 && force_shape_idx != 2)
    {
        GemvArgs g = gemv_args_single(A, trellis, C, c_fp32, suh, svh, m, k, n);
        int rc = launch_gemv(*ws, bits, cb, g, s, name);
        return rc ? rc : EXL3_AMD_TAG_GEMV;
    }
    // m > 8: input rotation into the caller's A_had (exl3_gemm_kernel.cuh writes it there too)
    if (suh && !A_had) return fail(EXL3_AMD_EINVAL, "%s: must supply A_had with suh", name);
    if (suh)
    {
        int rc = exl3k_had128(A, A_had, m, k, 0, suh, nullptr, 1.0f, 0, s);
        if (rc) return hip_fail(rc, name);
    }
    const uint16_t* A_rot = suh ? A_had : A;
    // Medium batches: the row-batched matrix-core GEMV in 16-row groups when it beats the tiled
    // GEMM.  Measured on MI355X (K = 2..4, k x n from 4096 x 1024 to 17408 x 5120, m = 16..192):
    // a 16-row group takes ~8 us + 0.37 ns per 1000 weights; a GEMM round (up to one tile per CU)
    // ~28 ns per k; with the split k, ~27 us + 28 ns per k of a split (input rotation, the
    // partial tiles and the fixup included).  The groups win at 16 rows, break even at 24-32.
    // force_shape_idx 1 takes the GEMV for any row count (16-row groups, each split in two
    // launches of at most 8 rows when the matrix-core GEMV is off or its plan does not fit).
    // The tiled GEMM splits k when its tiles fill at most half the CUs (LDS-DMA form): S ranges per
    // tile, as many as fill the CUs, at least 4 stages of 32 k each, the S fp32 partial tiles
    // within the workspace; the fixup kernel sums them in k order and runs the epilogue.
    const long blocks = (long) ((n + 255) / 256) * ((m + 255) / 256);
    const int staging = policy(EXL3_AMD_POLICY_GEMM_STAGING);
    int splits = 1;
    if (staging == 0 && 2 * blocks <= ws->num_cus)
    {
        const long tile_bytes = 256L * 256 * sizeof(float);
        long sp = std::min((long) ws->num_cus / blocks, (long) (k / 32) / 4);
        sp = std::min(sp, (long) (ws->partial_bytes / (tile_bytes * blocks)));
        splits = sp >= 2 ? (int) sp : 1;
    }
    bool groups = force_shape_idx == 1;
    if (force_shape_idx == 0 && gemv_mfma_mode() != 0)
    {
        const long rounds = (blocks + ws->num_cus - 1) / ws->num_cus;
        const double t_groups = ((m + 15) / 16) * (8.0 + 3.7e-7 * (double) n * k);
        const double t_gemm = splits > 1 ? 27.0 + 0.028 * k / splits : 0.028 * k * rounds;
        groups = t_groups < t_gemm;
    }
    if (groups)
    {
        const size_t elt = c_fp32 ? 4 : 2;
        for (int r0 = 0; r0 < m; r0 += 16)
        {
            GemvArgs g = gemv_args_single(A_rot + (size_t) r0 * k, trellis, (char*) C + (size_t) r0 * n * elt,
                                          c_fp32, nullptr, svh, std::min(16, m - r0), k, n);
            if (int rc = launch_gemv(*ws, bits, cb, g, s, name)) return rc;
        }
        return EXL3_AMD_TAG_GEMV;
    }
    GemmArgs gg;
    gg.A_rot = A_rot;
    gg.trellis = trellis; gg.C = C; gg.svh = svh;
    gg.m = m; gg.k = k; gg.n = n; gg.c_fp32 = c_fp32 ? 1 : 0;
    gg.reg_staging = staging == EXL3_AMD_GEMM_STAGING_REGS;
    gg.splits = splits;
    gg.part = ws->partials;
    int rc = dispatch_gemm(bits, cb, gg, s);
    return rc ? hip_fail(rc, name) : EXL3_AMD_TAG_GEMM;
}

}  // namespace

extern "C" {

int exl3_amd_gemm(const uint16_t* A, const uint16_t* trellis, void* C, int c_fp32,
                  const uint16_t* suh, uint16_t* A_had, const uint16_t* svh,
                  int m, int k, int n, float K, int mcg, int mul1, int force_shape_idx,
                  void* stream)
{
    return gemm_impl(nullptr, A, trellis, C, c_fp32, suh, A_had, svh, m, k, n, K, mcg, mul1, force_shape_idx, stream,
                     "exl3_gemm");
}

int exl3_amd_gemm_noalloc(const uint16_t* A, const uint16_t* trellis, void* C, int c_fp32,
                          const uint16_t* suh, uint16_t* A_had, const uint16_t* svh,
                          int m, int k, int n, float K, int mcg, int mul1, int force_shape_idx,
                          void* stream)
{
    g_last_error.clear();
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(EXL3_AMD_EHIP, "hipGetDevice failed");
    if (int rc = noalloc_setup(dev)) return rc;
    const NoAllocState& st = g_noalloc[dev];
    Workspace w;
    w.partials = (float*) st.ptr;
    w.partial_bytes = NOALLOC_PARTIAL_BYTES;
    w.counters = (int*) (st.ptr + NOALLOC_PARTIAL_BYTES);
    w.counter_ints = NOALLOC_COUNTER_INTS;
    w.sink = (const uint32_t*) (st.ptr + NOALLOC_PARTIAL_BYTES + NOALLOC_COUNTER_INTS * sizeof(int));
    w.num_cus = st.num_cus;
    // the XCD-local hand-off only where exl3_amd_init (or an earlier call of another entry point)
    // has already verified the dispatch order; otherwise the finish kernel sums the partials
    xcd_service(dev, (hipStream_t) stream);
    w.num_xcd = g_dev[dev].ready ? g_dev[dev].num_xcd : 0;
    w.alarm = g_dev[dev].ready ? g_dev[dev].alarm_dev : nullptr;
    return gemm_impl(&w, A, trellis, C, c_fp32, suh, A_had, svh, m, k, n, K, mcg, mul1, force_shape_idx, stream,
                     "exl3_gemm_noalloc");
}

static int mgemm_impl(const uint16_t* A, int bszm_in, int m, int k,
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
                   const float* in_sq, const uint16_t* in_w, float in_eps, uint16_t* in_r,
                   void* stream)
{
    (void) A_had; (void) force_num_sms;
    g_last_error.clear();
    int bits, half, cb;
    if (int rc = parse_K(K, mcg != 0, mul1 != 0, &bits, &half, &cb, "exl3_mgemm")) return rc;
    if (bszm_in < 1 || bszm_out < 1 || m < 0 || k < 0 || n < 0 || num_B < 0)
        return fail(EXL3_AMD_EINVAL, "exl3_mgemm: bad batch or size");
    if (!A || !B || !suh || !svh || (!C && !c_ptrs)) return fail(EXL3_AMD_EINVAL, "exl3_mgemm: null pointer");
    const bool sliced = had_src_list != nullptr;
    if (!sliced && (num_suh != num_B || num_svh != num_B))
        return fail(EXL3_AMD_EINVAL, "exl3_mgemm: B, suh and svh tables must have the same length");
    if (sliced && num_svh != num_B) return fail(EXL3_AMD_EINVAL, "exl3_mgemm: B and svh tables must have the same length");
    if (size_n_list)
    {
        if (!c_ptrs) return fail(EXL3_AMD_EINVAL, "exl3_mgemm: size_n_list requires c_ptrs");
        if (!(num_tokens == 1 && min_index < 0 && !weights))
            return fail(EXL3_AMD_EINVAL, "exl3_mgemm: per-matrix widths incompatible with multi-token/filtering/weights");
        bszm_out = num_c_ptrs;
    }
    else if (c_ptrs) return fail(EXL3_AMD_EINVAL, "exl3_mgemm: c_ptrs requires size_n_list");
    int bszm = bszm_in > bszm_out ? bszm_in : bszm_out;
    if (sliced)
    {
        if (!(size_n_list && c_ptrs && n_stride_list))
            return fail(EXL3_AMD_EINVAL, "exl3_mgemm: sliced mode requires size_n_list, c_ptrs and n_stride_list");
        if (!(bszm_in == 1 && !indices && !weights && num_tokens == 1 && min_index < 0))
            return fail(EXL3_AMD_EINVAL, "exl3_mgemm: sliced mode is single-input, unfiltered and single-token");
        if (num_had_src_list < bszm_out || num_n_stride < bszm_out)
            return fail(EXL3_AMD_EINVAL, "exl3_mgemm: had_src_list / n_stride_list must have one entry per slice");
        if (!(num_had_src > 0 && num_suh >= num_had_src))
            return fail(EXL3_AMD_EINVAL, "exl3_mgemm: sliced mode needs one suh entry per source");
    }
    else if (n_stride_list) return fail(EXL3_AMD_EINVAL, "exl3_mgemm: n_stride_list requires had_src_list");
    const int64_t had_slabs = sliced ? num_had_src : bszm;
    if (a_had_numel < had_slabs * (int64_t) m * k) return fail(EXL3_AMD_EINVAL, "exl3_mgemm: A_had must hold bszm * m * k elements");
    if (indices)
    {
        if (!(num_indices <= bszm_in || num_indices <= bszm_out))
            return fail(EXL3_AMD_EINVAL, "mgemm: too many indices for tensor batch");
        if (bszm_in > num_indices) bszm_in = num_indices;
        if (bszm_out > num_indices) bszm_out = num_indices;
    }
    bszm = bszm_in > bszm_out ? bszm_in : bszm_out;
    if (k % 16) return fail(EXL3_AMD_EINVAL, "exl3_mgemm: k must be a multiple of 16");
    if (n % 128) return fail(EXL3_AMD_EINVAL, "exl3_mgemm: n must be a multiple of 128");
    if (num_tokens < 1) return fail(EXL3_AMD_EINVAL, "exl3_mgemm: num_tokens must be positive");
    if (weights && bszm % num_tokens) return fail(EXL3_AMD_EINVAL, "exl3_mgemm: slots must split evenly into token groups");
    if (min_index >= 0 && !indices) return fail(EXL3_AMD_EINVAL, "exl3_mgemm: index range filtering requires indices");
    if (min_index >= 0 && bszm > MGEMM_MAX_FILTER)
        return fail(EXL3_AMD_EINVAL, "exl3_mgemm: range filtering supports at most %d slots", MGEMM_MAX_FILTER);
    if (force_shape_idx > 2) return fail(EXL3_AMD_EINVAL, "exl3_mgemm: bad force_shape_idx %d", force_shape_idx);
    if (m == 0 || n == 0 || bszm == 0) return EXL3_AMD_TAG_GEMV;
    if (k == 0) return fail(EXL3_AMD_EINVAL, "exl3_mgemm: k must be positive");
    if (k % 128) return fail(EXL3_AMD_EUNSUPPORTED, "exl3_mgemm: k %% 128 != 0 is not implemented in this build");

    DeviceState* d;
    if (int rc = current_device(&d, stream)) return rc;
    hipStream_t s = (hipStream_t) stream;

    GemvArgs g;
    memset(&g, 0, sizeof(g));
    g.A = A; g.C = C; g.m = m; g.k = k; g.n = n; g.c_fp32 = c_fp32 ? 1 : 0;
    g.B_list = B; g.suh_list = suh; g.svh_list = svh;
    g.indices = indices; g.weights = weights;
    g.size_n = size_n_list; g.c_list = c_ptrs; g.n_stride = n_stride_list; g.had_src = had_src_list;
    g.bszm_in = bszm_in; g.bszm = bszm; g.num_tokens = num_tokens;
    if (min_index >= 0)
    {
        int rc = exl3k_mgemm_filter(indices, weights, bszm, min_index, max_index, num_tokens, d->filt_idx, d->filt_w, s);
        if (rc) return hip_fail(rc, "exl3_mgemm");
        g.indices = d->filt_idx;
        if (weights) g.weights = d->filt_w;
    }
    if (in_w)
    {
        // consumer half of a split residual norm: one row forms its input in the M = 1 stream
        // kernel (launch_gemv falls back for other plans); more rows normalise into in_r first
        if (m == 1)
        {
            g.in_sq = in_sq; g.in_w = in_w; g.in_eps = in_eps; g.in_r = in_r;
        }
        else
        {
            if (int rc = exl3k_norm_sq(A, in_sq, in_w, in_r, m, k, in_eps, s)) return hip_fail(rc, "exl3_mgemm_norm_in");
            g.A = in_r;
        }
    }
    // more than 8 rows: the GEMV in 16-row groups (slab strides stay those of all m rows); a
    // group runs on the row-batched matrix-core kernel, or as two launches of at most 8 rows on
    // the LDS kernel (launch_gemv)
    g.slab_m = m;
    const int group = 16;
    for (int r0 = 0; r0 < m; r0 += group)
    {
        GemvArgs gr = g;
        gr.m = std::min(group, m - r0);
        gr.row0 = r0;
        if (int rc = launch_gemv(ws_of(d), bits, cb, gr, s, "exl3_mgemm")) return rc;
    }
    return EXL3_AMD_TAG_GEMV;
}

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
                   void* stream)
{
    return mgemm_impl(A, bszm_in, m, k, B, num_B, C, bszm_out, n, c_fp32, suh, num_suh, A_had, a_had_numel, svh, num_svh,
                      indices, num_indices, weights, K, force_shape_idx, mcg, mul1, min_index, max_index, force_num_sms,
                      num_tokens, size_n_list, c_ptrs, num_c_ptrs, n_stride_list, num_n_stride, had_src_list,
                      num_had_src_list, num_had_src, nullptr, nullptr, 0.0f, nullptr, stream);
}

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
                           void* stream)
{
    g_last_error.clear();
    if (!sq || !w || !r) return fail(EXL3_AMD_EINVAL, "exl3_mgemm_norm_in: null pointer");
    if (((uintptr_t) h | (uintptr_t) sq | (uintptr_t) w | (uintptr_t) r) & 3)
        return fail(EXL3_AMD_EINVAL, "exl3_mgemm_norm_in: h, sq, w and r must be 4-byte aligned");
    if (bszm_in != 1) return fail(EXL3_AMD_EINVAL, "exl3_mgemm_norm_in: the input must be one slab (broadcast)");
    if (k > 64 * SQ_SCALE_MAX_PER_LANE * 128 || m > 65535)
        return fail(EXL3_AMD_EINVAL, "exl3_mgemm_norm_in: k above %d or more than 65535 rows", 64 * SQ_SCALE_MAX_PER_LANE * 128);
    return mgemm_impl(h, bszm_in, m, k, B, num_B, C, bszm_out, n, c_fp32, suh, num_suh, A_had, a_had_numel, svh, num_svh,
                      nullptr, 0, nullptr, K, -1, mcg, mul1, -1, -1, 0, 1, size_n_list, c_ptrs, num_c_ptrs,
                      n_stride_list, num_n_stride, had_src_list, num_had_src_list, num_had_src, sq, w, eps, r, stream);
}

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
                      void* stream)
{
    (void) gu_g; (void) gu_u; (void) gu_f32; (void) d_out;
    g_last_error.clear();
    // exl3_moe_coop.cu:185-305 (prepare + run), in the reference's order
    if (!x || !sel || !rw || !out || !ctr || !had_g || !had_u || !act_out)
        return fail(EXL3_AMD_EINVAL, "exl3_moe_coop: null pointer");
    if (!g_trellis || !g_suh || !g_svh || !u_trellis || !u_suh || !u_svh || !d_trellis || !d_suh || !d_svh)
        return fail(EXL3_AMD_EINVAL, "exl3_moe_coop: pointer tables must be contiguous int64");
    if (mcg && mul1) return fail(EXL3_AMD_EINVAL, "exl3_moe_coop: specified both mcg and mul1");
    if (!(Kg >= 1 && Kg <= 8 && Ku >= 1 && Ku <= 8 && Kd >= 1 && Kd <= 8))
        return fail(EXL3_AMD_EINVAL, "exl3_moe_coop: K out of range");
    if (gated && Kg != Ku) return fail(EXL3_AMD_EINVAL, "exl3_moe_coop: gate and up must share a bit width");
    if (act < 0 || act > 3) return fail(EXL3_AMD_EINVAL, "exl3_moe_coop: unknown activation");
    if (!(Hi % 128 == 0 && I % 128 == 0 && Ho % 128 == 0 && H_out <= Ho && Hi > 0 && I > 0 && Ho > 0))
        return fail(EXL3_AMD_EINVAL, "exl3_moe_coop: Hi/I/Ho shape");
    int64_t sm = had_g_numel / Hi;
    sm = std::min<int64_t>(sm, had_u_numel / Hi);
    sm = std::min<int64_t>(sm, gu_numel / I);
    sm = std::min<int64_t>(sm, act_out_numel / I);
    sm = std::min<int64_t>(sm, d_out_numel / Ho);
    if (sm < 1 || sm > 256) return fail(EXL3_AMD_EINVAL, "exl3_moe_coop: scratch must hold 1..256 slots");
    const int slots_max = (int) sm;
    const int64_t ctr_len = (int64_t) slots_max * (I / 128) + (int64_t) rows_max * (Ho / 128) + 2 + (slots_max + 1) + slots_max;
    if (ctr_numel < ctr_len) return fail(EXL3_AMD_EINVAL, "exl3_moe_coop: counter scratch too small");
    if ((bits_g || bits_u || bits_d) && !(bits_g && bits_u && bits_d))
        return fail(EXL3_AMD_EINVAL, "exl3_moe_coop: give all three bit width tables or none");
    if (bsz < 0 || topk < 1) return fail(EXL3_AMD_EINVAL, "exl3_moe_coop: sel/rw must be (bsz, topk)");
    if (!(H % 4 == 0 && H <= Hi)) return fail(EXL3_AMD_EINVAL, "exl3_moe_coop: H/Hi shape");
    const int slots = bsz * topk;
    if (!(slots <= slots_max && bsz <= rows_max)) return fail(EXL3_AMD_EINVAL, "exl3_moe_coop: batch exceeds the scratch");
    if (!(min_expert < 0 || max_expert - min_expert <= n_local))
        return fail(EXL3_AMD_EINVAL, "exl3_moe_coop: expert range exceeds tables");
    if (sh_out)
    {
        if (H_out != H) return fail(EXL3_AMD_EINVAL, "exl3_moe_coop: shared expert output width must match the routed output");
        if (sh_gate_w && !(sh_gate_n == H && H % 2 == 0)) return fail(EXL3_AMD_EINVAL, "exl3_moe_coop: shared gate width");
    }
    const bool dyn = bits_g != nullptr;
    if (dyn && !mul1) return fail(EXL3_AMD_EINVAL, "exl3_moe_coop: mixed bit widths require the mul1 codebook");
    const float Kgu = gated ? Kg : Ku;
    int kgu_code, kd_code, half_, cbk;              // rate codes (integer, or 16 + b for b + 1/2)
    if (int rc = parse_K(Kgu, mcg, mul1, &kgu_code, &half_, &cbk, "exl3_moe_coop")) return rc;
    if (int rc = parse_K(Kd, mcg, mul1, &kd_code, &half_, &cbk, "exl3_moe_coop")) return rc;
    if (bsz == 0) return 0;

    DeviceState* d;
    if (int rc = current_device(&d, stream)) return rc;

    MoeArgs a;
    memset(&a, 0, sizeof(a));
    a.x = x; a.x_stride = x_stride; a.sel = sel; a.rw = rw;
    a.bsz = bsz; a.topk = topk; a.H = H; a.Hi = Hi; a.I = I; a.Ho = Ho; a.H_out = H_out;
    a.min_expert = min_expert; a.max_expert = max_expert;
    a.g_trellis = g_trellis; a.g_suh = g_suh; a.g_svh = g_svh;
    a.u_trellis = u_trellis; a.u_suh = u_suh; a.u_svh = u_svh;
    a.d_trellis = d_trellis; a.d_suh = d_suh; a.d_svh = d_svh;
    a.g_bias = g_bias; a.u_bias = u_bias; a.d_bias = d_bias;
    a.g_bits = bits_g; a.u_bits = bits_u; a.d_bits = bits_d;
    a.K_gu = kgu_code; a.K_d = kd_code;
    a.act = act; a.act_limit = act_limit; a.gated = gated ? 1 : 0;
    a.had_g = had_g; a.had_u = had_u; a.act_out = act_out;
    a.runs = ctr + (int64_t) slots_max * (I / 128) + (int64_t) rows_max * (Ho / 128);
    a.slots_max = slots_max;
    a.out = out; a.out_stride = out_stride;
    a.sh_out = sh_out; a.sh_gate_w = sh_out ? sh_gate_w : nullptr;

    // work split: k-splits so every workgroup holds at most EXL3_MOE_SBMAX k-slices and the grid
    // (sized for one run per slot) reaches a few workgroups per CU
    const int nproj = gated ? 2 : 1;
    // 2 workgroups per CU: the one-token batch (8 slots) then splits gate/up and down k in 2
    // (measured 1, 2, 4, 8 per CU: 51.9, 51.6, 53.6, 68.4 us)
    const long target = 2L * d->num_cus;
    auto pick = [&](int KS, long base) {
        int S = (KS + EXL3_MOE_SBMAX - 1) / EXL3_MOE_SBMAX;
        while (base * S < target && KS / (S + 1) >= 8) ++S;
        return S;
    };
    a.splits_a = pick(Hi / 16, (long) slots * (I / 128) * nproj);
    a.splits_b = pick(I / 16, (long) slots * (Ho / 128));
    const size_t pa = (size_t) 2 * a.splits_a * slots * I, pb = (size_t) a.splits_b * slots * Ho;
    if ((pa + pb) * 4 > WS_PARTIAL_BYTES) return fail(EXL3_AMD_EUNSUPPORTED, "exl3_moe_coop: batch exceeds the library workspace");
    a.part_a = d->partials;
    a.part_b = d->partials + pa;
    const size_t ca = (size_t) slots * (I / 128) * 32, cb_ = (size_t) bsz * (Ho / 128) * 32;
    if (ca + cb_ > WS_COUNTERS) return fail(EXL3_AMD_EUNSUPPORTED, "exl3_moe_coop: batch exceeds the counter workspace");
    a.ctr_a = d->counters;
    a.ctr_b = d->counters + ca;
    a.xcd = (d->num_xcd > 0 && (I / 128) % d->num_xcd == 0 && (Ho / 128) % d->num_xcd == 0 &&
             (long) nproj * a.splits_a <= XCD_MAX_ARRIVALS && (long) topk * a.splits_b <= XCD_MAX_ARRIVALS) ? d->num_xcd : 0;
    a.xg = xcd_guard(d->alarm_dev);
    a.epi_serial = policy(EXL3_AMD_POLICY_MOE_EPILOGUE) == EXL3_AMD_MOE_EPILOGUE_SERIAL;

    const int cb = mcg ? 1 : (mul1 ? 2 : 0);
    hipStream_t s = (hipStream_t) stream;
    int rc = cb == 0 ? exl3k_moe_cb0(a, s) : cb == 1 ? exl3k_moe_cb1(a, s) : exl3k_moe_cb2(a, s);
    return rc ? hip_fail(rc, "exl3_moe_coop") : 0;
}


int exl3_amd_moe_max_concurrency(int device)
{
    g_last_error.clear();
    DeviceState* d;
    if (int rc = init_device(device, &d)) return rc;
    return d->num_cus / 8;                           // exl3_moe.cu:15-19 (MOE_SMS_PER_EXPERT = 8)
}

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
                 void* stream)
{
    g_last_error.clear();
    // exl3_moe.cu:186-323, in the reference's order
    if (num_active == 0) return 0;
    if (output_scratch)
    {
        if (!fused_base) return fail(EXL3_AMD_EINVAL, "exl3_moe: output_scratch needs fused_base");
        if (scratch_cols != hidden_dim) return fail(EXL3_AMD_EINVAL, "exl3_moe: output_scratch must be [slots, hidden]");
    }
    if (!hidden_state || !output_state || !expert_count || !token_sorted || !weight_sorted || !temp_state_g ||
        !temp_state_u || !temp_intermediate_g || !temp_intermediate_u)
        return fail(EXL3_AMD_EINVAL, "exl3_moe: null pointer");
    if (bsz < 1 || expert_count_len < 1 || num_assign % bsz != 0)
        return fail(EXL3_AMD_EINVAL, "exl3_moe: token_sorted must hold bsz * num_experts_per_tok entries");
    const int num_experts = expert_count_len - 1;
    if (concurrency < 1 || max_tokens_per_expert < 1 || intermediate_dim < 1)
        return fail(EXL3_AMD_EINVAL, "exl3_moe: temp buffer shapes");
    if (!(gate_mcg == up_mcg && up_mcg == down_mcg && gate_mul1 == up_mul1 && up_mul1 == down_mul1))
        return fail(EXL3_AMD_EINVAL, "MoE kernel: gate/up/down must share the same codebook");
    if (gate_mcg == gate_mul1) return fail(EXL3_AMD_EINVAL, "MoE kernel: Only mcg and mul1 codebooks are supported");
    auto k2 = [](float K) { return (int) (2.0f * K); };
    const int K2g = k2(K_gate), K2u = k2(K_up), K2d = k2(K_down);
    if (!gate_mul1 && (K2g % 2 || K2u % 2 || K2d % 2))
        return fail(EXL3_AMD_EINVAL, "exl3_moe: half-integer bitrates require the mul1 codebook");
    if (bits_g || bits_u || bits_d)
    {
        if (!(bits_g && bits_u && bits_d)) return fail(EXL3_AMD_EINVAL, "exl3_moe: give all three bit width tables or none");
        if (bits_len < num_experts)
            return fail(EXL3_AMD_EINVAL, "exl3_moe: bit width tables must be contiguous uint8, one entry per expert");
        if (!gate_mul1) return fail(EXL3_AMD_EINVAL, "exl3_moe: mixed bit widths require the mul1 codebook");
    }
    if (!gate_ptrs_trellis || !gate_ptrs_suh || !gate_ptrs_svh || !up_ptrs_trellis || !up_ptrs_suh ||
        !up_ptrs_svh || !down_ptrs_trellis || !down_ptrs_suh || !down_ptrs_svh)
        return fail(EXL3_AMD_EINVAL, "exl3_moe: null pointer table");
    if (num_ptrs != num_experts) return fail(EXL3_AMD_EINVAL, "Number of gate tensors doesn't match num_experts");

    DeviceState* d;
    if (int rc = current_device(&d, stream)) return rc;
    if (concurrency * 8 > d->num_cus) return fail(EXL3_AMD_EINVAL, "Concurrency too high for device num_sms");
    if (m_tile > 16)
    {
        if (!gate_mul1) return fail(EXL3_AMD_EINVAL, "exl3_moe: row tiles above 16 are instantiated for the mul1 codebook only");
        if (max_tokens_per_expert < m_tile) return fail(EXL3_AMD_EINVAL, "exl3_moe: temp buffers hold fewer rows than the tile");
    }
    // this build's limits: 128-multiples (every row is rotated in 128-chunks), the plan's expert count
    if (hidden_dim % 128 || intermediate_dim % 128)
        return fail(EXL3_AMD_EUNSUPPORTED, "exl3_moe: hidden and intermediate sizes must be multiples of 128");
    // bits_k.cuh:12-27: integer 1..8, or 1.5 / 2.5 / 3.5
    auto k2_ok = [](int K2) { return (K2 % 2 == 0 && K2 >= 2 && K2 <= 16) || K2 == 3 || K2 == 5 || K2 == 7; };
    if (!bits_g && !(k2_ok(K2g) && k2_ok(K2u) && k2_ok(K2d)))
        return fail(EXL3_AMD_EINVAL, "exl3_moe: bitrate out of range");
    auto rate = [](int K2) { return K2 % 2 ? 16 + K2 / 2 : K2 / 2; };     // the kernels' rate code
    if (num_experts > 4096) return fail(EXL3_AMD_EUNSUPPORTED, "exl3_moe: more than 4096 experts");

    const int64_t pool64 = (int64_t) concurrency * max_tokens_per_expert;
    const int pool = (int) std::min<int64_t>(pool64, (int64_t) num_assign);   // rows a pass can hold
    // rows per MFMA tile from the mean rows per expert: one tile covers most experts, with
    // little padding (the weights are decoded once per tile).  LDS-tiled kernel, measured on
    // MI355X, 256 experts 4096 -> 2048 -> 4096, top-8: best tile 64 up to a mean of 32 rows,
    // 128 at 64, 256 at 128
    const int mean_rows = num_assign / std::max(num_experts, 1);
    // GEMM kernel: the register-decode moeg_kernel (default) or the LDS-tiled gemm_kernel
    // (policy EXL3_AMD_POLICY_MOE_GEMM = EXL3_AMD_MOE_GEMM_LDS).  moeg rows per tile: one tile per
    // expert for most experts
    const bool reg_gemm = policy(EXL3_AMD_POLICY_MOE_GEMM) != EXL3_AMD_MOE_GEMM_LDS;
    // moeg: the smallest tile holding ~1.5x the mean rows (the largest expert, for top-k routing
    // of random tokens).  Measured, 256 experts 4096 -> 2048 -> 4096, top-8: T = 512 (mean 16,
    // max 27) best at 32; T = 2048 (mean 64, max 91) best at 96: 2.32 ms against 2.49 at 64 and
    // 2.54 at 128 (fewer tiles read each expert's weights fewer times; 96 keeps 3 waves per SIMD)
    const int want = mean_rows * 3 / 2;
    int tile_rows = reg_gemm ? (want <= 32 ? 32 : (want <= 64 ? 64 : (want <= 96 ? 96 : 128)))
                             : (mean_rows <= 40 ? 64 : (mean_rows <= 96 ? 128 : 256));
    // policy EXL3_AMD_POLICY_MOE_TILE_ROWS: a forced tile height (tests cover every instance)
    {
        const int v = policy(EXL3_AMD_POLICY_MOE_TILE_ROWS);
        if (reg_gemm ? (v == 32 || v == 64 || v == 96 || v == 128) : (v == 64 || v == 128 || v == 256)) tile_rows = v;
    }
    // persistent moeg workgroups: 4 per CU
    const int grid_wgs = d->num_cus * 4;
    const int rt_cap = pool / tile_rows + std::min(num_experts, pool) + 1;
    const size_t ps_floats = (size_t) pool * (2 * (hidden_dim / 128) + intermediate_dim / 128);
    // token-major output lists (atomic mode): starts, positions, build space, position -> row
    // (used when the per-call list build fits one workgroup's LDS; else the atomic output kernel)
    // (policy EXL3_AMD_POLICY_MOE_OUTPUT = EXL3_AMD_MOE_OUTPUT_ATOMIC forces the atomic output kernel)
    const bool tok_mode = !output_scratch && exl3k_moes_tokens_lds(bsz, num_assign) <= 150 * 1024
                          && policy(EXL3_AMD_POLICY_MOE_OUTPUT) != EXL3_AMD_MOE_OUTPUT_ATOMIC;
    const size_t tok_ints = tok_mode ? (size_t) (bsz + 1) + 2 * (size_t) num_assign : 0;
    const size_t ws_ints = (size_t) 3 * pool + 3 * (size_t) rt_cap + 3 * MOES_RATES * ((size_t) rt_cap + 1) + ps_floats
                         + tok_ints;
    if (ws_ints * 4 > WS_PARTIAL_BYTES) return fail(EXL3_AMD_EUNSUPPORTED, "exl3_moe: pool exceeds the library workspace");

    MoesArgs a;
    memset(&a, 0, sizeof(a));
    a.x = hidden_state; a.out = output_state; a.scratch = output_scratch; a.fused_base = fused_base;
    a.expert_count = expert_count; a.token_sorted = token_sorted; a.weight_sorted = weight_sorted;
    a.num_experts = num_experts; a.num_assign = num_assign; a.H = hidden_dim; a.I = intermediate_dim;
    a.max_tokens = max_tokens_per_expert; a.count_lo = count_lo; a.count_hi = count_hi;
    a.pool_rows = pool;
    a.ts_g = temp_state_g; a.ts_u = temp_state_u; a.ti_g = temp_intermediate_g; a.ti_u = temp_intermediate_u;
    a.g_trellis = gate_ptrs_trellis; a.g_suh = gate_ptrs_suh; a.g_svh = gate_ptrs_svh;
    a.u_trellis = up_ptrs_trellis; a.u_suh = up_ptrs_suh; a.u_svh = up_ptrs_svh;
    a.d_trellis = down_ptrs_trellis; a.d_suh = down_ptrs_suh; a.d_svh = down_ptrs_svh;
    a.bits_g = bits_g; a.bits_u = bits_u; a.bits_d = bits_d;
    a.K_g = rate(K2g); a.K_u = rate(K2u); a.K_d = rate(K2d);
    a.act = act_function; a.gated = act_function != 2;      // MOE_ACT_RELU2_NOGATE skips the gate
    a.act_limit = act_limit;
    int* ws = (int*) d->partials;
    a.rowinfo = ws;
    a.rt = ws + 3 * (size_t) pool;
    a.lists = a.rt + 3 * (size_t) rt_cap;
    a.counts = a.lists + 3 * MOES_RATES * (size_t) rt_cap;
    a.ps_g = (float*) (a.counts + 3 * MOES_RATES);
    a.ps_u = a.ps_g + (size_t) pool * (hidden_dim / 128);
    a.ps_d = a.ps_u + (size_t) pool * (hidden_dim / 128);
    a.rt_cap = rt_cap;
    a.tile_rows = tile_rows;
    a.bsz = bsz;
    if (tok_mode)
    {
        a.tok_start = (int*) (a.ps_d + (size_t) pool * (intermediate_dim / 128));
        a.tok_pos = a.tok_start + (bsz + 1);
        a.inv_row = a.tok_pos + num_assign;
    }

    typedef int (*group_fn)(const GemmGroupArgs&, int, hipStream_t);
    static const group_fn gfn_lds[MOES_RATES] = {
        exl3k_gemm_group_k1, exl3k_gemm_group_k2, exl3k_gemm_group_k3, exl3k_gemm_group_k4, exl3k_gemm_group_k5,
        exl3k_gemm_group_k6, exl3k_gemm_group_k7, exl3k_gemm_group_k8, exl3k_gemm_group_k17, exl3k_gemm_group_k18,
        exl3k_gemm_group_k19 };
    static const group_fn gfn_reg[MOES_RATES] = {
        exl3k_moeg_k1, exl3k_moeg_k2, exl3k_moeg_k3, exl3k_moeg_k4, exl3k_moeg_k5, exl3k_moeg_k6, exl3k_moeg_k7,
        exl3k_moeg_k8, exl3k_moeg_k17, exl3k_moeg_k18, exl3k_moeg_k19 };
    const group_fn* gfn = reg_gemm ? gfn_reg : gfn_lds;
    const int cb = gate_mul1 ? 2 : 1;
    hipStream_t s = (hipStream_t) stream;
    // one grouped launch per (phase, bitrate) that can occur: the list counts sit on the device
    auto gemm_phase = [&](int phase) -> int {
        for (int slot = 0; slot < MOES_RATES; ++slot)
        {
            const int K = moes_slot_rate(slot);
            GemmGroupArgs g;
            memset(&g, 0, sizeof(g));
            g.rt = a.rt;
            g.nrt = rt_cap;
            g.tile_rows = tile_rows;
            g.grid_wgs = grid_wgs;
            int mats = 0;
            auto add = [&](int m, const uint16_t* A, uint16_t* C, const uint64_t* tab, int Km, const float* ps) {
                if (bits_g ? K > 8 : Km != K) return;          // the tables hold integer widths
                g.A[mats] = A; g.C[mats] = C; g.tab[mats] = tab; g.psum[mats] = ps;
                g.list[mats] = a.lists + (size_t) (m * MOES_RATES + slot) * rt_cap;
                g.count[mats] = a.counts + m * MOES_RATES + slot;
                ++mats;
            };
            if (phase == 0)
            {
                if (a.gated) add(0, a.ts_g, a.ti_g, a.g_trellis, a.K_g, a.ps_g);
                add(1, a.ts_u, a.ti_u, a.u_trellis, a.K_u, a.ps_u);
                g.k = hidden_dim; g.n = intermediate_dim;
            }
            else
            {
                add(2, a.ti_g, a.ts_g, a.d_trellis, a.K_d, a.ps_d);
                g.k = intermediate_dim; g.n = hidden_dim;
            }
            if (!mats) continue;
            g.mats = mats;
            if (int rc = gfn[slot](g, cb, s)) return rc;
        }
        return 0;
    };
    const int cus = d->num_cus;
    if (a.tok_start)
        if (int rc = exl3k_moes_tokens(a, s)) return hip_fail(rc, "exl3_moe");
    for (int row0 = 0; row0 < num_assign; row0 += pool)
    {
        int rc = exl3k_moes_plan(a, row0, s);
        if (!rc) rc = exl3k_moes_gather(a, cus, s);
        if (!rc) rc = gemm_phase(0);
        if (!rc) rc = exl3k_moes_act(a, cus, s);
        if (!rc) rc = gemm_phase(1);
        if (!rc) rc = exl3k_moes_out(a, cus, s);
        if (rc) return hip_fail(rc, "exl3_moe");
    }
    return 0;
}

int exl3_amd_moe_gather(float* output_state, int tokens, int hidden_dim,
                        const float* output_scratch, int scratch_cols,
                        const int64_t* flat_expert, int num_assign, const int64_t* inv_order,
                        const int64_t* expert_start, int expert_start_len,
                        const int64_t* slot_base, int slot_base_len,
                        const int64_t* slot_kind, int num_experts,
                        const uint16_t* weight_sorted, void* stream)
{
    g_last_error.clear();
    // exl3_moe.cu:480-527
    if (!output_state || !output_scratch || !flat_expert || !inv_order || !expert_start || !slot_base ||
        !slot_kind || !weight_sorted)
        return fail(EXL3_AMD_EINVAL, "exl3_moe_gather: null pointer");
    if (scratch_cols != hidden_dim) return fail(EXL3_AMD_EINVAL, "exl3_moe_gather: output_scratch must be [slots, hidden]");
    if (tokens < 0 || (tokens > 0 && num_assign % tokens != 0)) return fail(EXL3_AMD_EINVAL, "exl3_moe_gather: assignments / tokens");
    if (!(slot_base_len >= num_experts && expert_start_len >= num_experts)) return fail(EXL3_AMD_EINVAL, "exl3_moe_gather: table sizes");
    if (!tokens) return 0;
    const int topk = num_assign / tokens;
    if (topk > 32) return fail(EXL3_AMD_EINVAL, "exl3_moe_gather: top-k too large");
    DeviceState* d;
    if (int rc = current_device(&d, stream)) return rc;
    MoesGatherArgs g;
    g.out = output_state; g.scratch = output_scratch; g.flat_expert = flat_expert; g.inv_order = inv_order;
    g.expert_start = expert_start; g.slot_base = slot_base; g.slot_kind = slot_kind; g.weight_sorted = weight_sorted;
    g.tokens = tokens; g.H = hidden_dim; g.topk = topk; g.num_experts = num_experts;
    int rc = exl3k_moes_sum(g, (hipStream_t) stream);
    return rc ? hip_fail(rc, "exl3_moe_gather") : 0;
}


int exl3_amd_rms_norm_res(const uint16_t* x, const uint16_t* r, const uint16_t* w, uint16_t* y, uint16_t* n,
                          int64_t rows, int dim, float eps, void* stream)
{
    g_last_error.clear();
    // amp_torch.cpp:10106-10131 and amp_kernels.cu:371-381
    if (rows < 0 || dim < 0) return fail(EXL3_AMD_EINVAL, "rms_norm_res: negative size");
    if (rows == 0 || dim == 0) return 0;
    if (dim % 4) return fail(EXL3_AMD_EINVAL, "rms_norm_res: last dim (%d) must be a multiple of 4", dim);
    if (!x || !r || !w || !y || !n) return fail(EXL3_AMD_EINVAL, "rms_norm_res: null pointer");
    if (((uintptr_t) x | (uintptr_t) r | (uintptr_t) w | (uintptr_t) y | (uintptr_t) n) & 7)
        return fail(EXL3_AMD_EINVAL, "rms_norm_res: tensors must be 8-byte aligned");
    if (rows > 0x7fffffff) return fail(EXL3_AMD_EINVAL, "rms_norm_res: too many rows");
    DeviceState* d;
    if (int rc = current_device(&d, stream)) return rc;
    int rc = exl3k_rms_norm_res(x, r, w, y, n, (long) rows, dim, eps, (hipStream_t) stream);
    return rc ? hip_fail(rc, "rms_norm_res") : 0;
}

int exl3_amd_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* out, int64_t numel, void* stream)
{
    g_last_error.clear();
    if (numel <= 0) return 0;
    if (!g || !u || !out) return fail(EXL3_AMD_EINVAL, "silu_mul: null pointer");
    DeviceState* d;
    if (int rc = current_device(&d, stream)) return rc;
    int rc = exl3k_silu_mul(g, u, out, (long) numel, (hipStream_t) stream);
    return rc ? hip_fail(rc, "silu_mul") : 0;
}

int exl3_amd_gemm_silu_mul(const uint16_t* gate, const uint16_t* up, uint16_t* act,
                           const uint16_t* trellis, void* C, int c_fp32,
                           const uint16_t* suh, uint16_t* A_had, const uint16_t* svh,
                           int m, int k, int n, float K, int mcg, int mul1, void* stream)
{
    g_last_error.clear();
    int bits, half, cb;
    if (int rc = parse_K(K, mcg, mul1, &bits, &half, &cb, "exl3_gemm")) return rc;
    if (m < 0 || k < 0 || n < 0) return fail(EXL3_AMD_EINVAL, "exl3_gemm: negative size");
    if (m == 0 || n == 0) return EXL3_AMD_TAG_GEMV;
    if (!gate || !up || !act || !trellis || !C) return fail(EXL3_AMD_EINVAL, "exl3_gemm_silu_mul: null pointer");
    if (k % 16) return fail(EXL3_AMD_EINVAL, "exl3_gemm: k must be a multiple of 16");
    if (n % 128) return fail(EXL3_AMD_EINVAL, "exl3_gemm: n must be a multiple of 128");
    if (k == 0) return fail(EXL3_AMD_EINVAL, "exl3_gemm: k must be positive");
    if (k % 128) return fail(EXL3_AMD_EUNSUPPORTED, "exl3_gemm: k %% 128 != 0 is not implemented in this build");
    DeviceState* d;
    if (int rc = current_device(&d, stream)) return rc;
    hipStream_t s = (hipStream_t) stream;
    if (m == 1)
    {
        GemvArgs g = gemv_args_single(gate, trellis, C, c_fp32, suh, svh, m, k, n);
        GemvArgs probe = g;
        if (!gemv_plan(m, k, n, 1, d->num_cus, probe, WS_PARTIAL_BYTES) && probe.stream_m1 == 1)
        {
            g.A_up = up;                             // silu(gate) * up formed in the input load
            int rc = launch_gemv(ws_of(d), bits, cb, g, s, "exl3_gemm_silu_mul");
            return rc ? rc : EXL3_AMD_TAG_GEMV;
        }
    }
    if (int rc = exl3k_silu_mul(gate, up, act, (long) m * k, s)) return hip_fail(rc, "exl3_gemm_silu_mul");
    return exl3_amd_gemm(act, trellis, C, c_fp32, suh, A_had, svh, m, k, n, K, mcg, mul1, 0, stream);
}


int exl3_amd_gemm_norm(const uint16_t* A, const uint16_t* up, uint16_t* act, const uint16_t* trellis, uint16_t* C,
                       const uint16_t* suh, uint16_t* A_had, const uint16_t* svh,
                       int m, int k, int n, float K, int mcg, int mul1,
                       uint16_t* h, const uint16_t* w, uint16_t* r, float eps, void* stream)
{
    g_last_error.clear();
    int bits, half, cb;
    if (int rc = parse_K(K, mcg, mul1, &bits, &half, &cb, "exl3_gemm")) return rc;
    if (m < 1 || k < 1 || n < 1) return fail(EXL3_AMD_EINVAL, "exl3_gemm_norm: sizes must be positive");
    if (k % 16) return fail(EXL3_AMD_EINVAL, "exl3_gemm: k must be a multiple of 16");
    if (n % 128) return fail(EXL3_AMD_EINVAL, "exl3_gemm: n must be a multiple of 128");
    if (k % 128) return fail(EXL3_AMD_EUNSUPPORTED, "exl3_gemm: k %% 128 != 0 is not implemented in this build");
    if (!A || !trellis || !C || !h || !w || !r || (up && !act)) return fail(EXL3_AMD_EINVAL, "exl3_gemm_norm: null pointer");
    if (((uintptr_t) C | (uintptr_t) h | (uintptr_t) w | (uintptr_t) r) & 15)
        return fail(EXL3_AMD_EINVAL, "exl3_gemm_norm: C, h, w and r must be 16-byte aligned");
    DeviceState* d;
    if (int rc = current_device(&d, stream)) return rc;
    hipStream_t s = (hipStream_t) stream;
    if (m == 1)
    {
        GemvArgs g = gemv_args_single(A, trellis, C, 0, suh, svh, m, k, n);
        GemvArgs probe = g;
        const bool plan_ok = !gemv_plan(m, k, n, 1, d->num_cus, probe, WS_PARTIAL_BYTES) && probe.stream_m1 == 1;
        const int chunks = n / 128;
        const bool handoff = probe.slots == 1 || (d->num_xcd > 0 && chunks % d->num_xcd == 0 && chunks * 32 <= (int) (WS_COUNTERS / 2));
        if (plan_ok && handoff)
        {
            g.A_up = up;
            g.norm_h = h; g.norm_w = w; g.norm_r = r; g.norm_eps = eps;
            g.norm_ctr = d->counters + WS_NORM_CTR;
            int rc = launch_gemv(ws_of(d), bits, cb, g, s, "exl3_gemm_norm");
            return rc ? rc : EXL3_AMD_TAG_GEMV;
        }
    }
    int tag = up ? exl3_amd_gemm_silu_mul(A, up, act, trellis, C, 0, suh, A_had, svh, m, k, n, K, mcg, mul1, stream)
                 : exl3_amd_gemm(A, trellis, C, 0, suh, A_had, svh, m, k, n, K, mcg, mul1, 0, stream);
    if (tag < 0) return tag;
    if (int rc = exl3_amd_rms_norm_res(h, C, w, h, r, m, n, eps, stream)) return rc;
    return tag;
}

int exl3_amd_gemm_res(const uint16_t* A, const uint16_t* up, uint16_t* act, const uint16_t* trellis, uint16_t* C,
                      const uint16_t* suh, uint16_t* A_had, const uint16_t* svh,
                      int m, int k, int n, float K, int mcg, int mul1,
                      uint16_t* h, float* sq, void* stream)
{
    g_last_error.clear();
    int bits, half, cb;
    if (int rc = parse_K(K, mcg, mul1, &bits, &half, &cb, "exl3_gemm")) return rc;
    if (m < 1 || k < 1 || n < 1) return fail(EXL3_AMD_EINVAL, "exl3_gemm_res: sizes must be positive");
    if (k % 16) return fail(EXL3_AMD_EINVAL, "exl3_gemm: k must be a multiple of 16");
    if (n % 128) return fail(EXL3_AMD_EINVAL, "exl3_gemm: n must be a multiple of 128");
    if (k % 128) return fail(EXL3_AMD_EUNSUPPORTED, "exl3_gemm: k %% 128 != 0 is not implemented in this build");
    if (!A || !trellis || !C || !h || !sq || (up && !act)) return fail(EXL3_AMD_EINVAL, "exl3_gemm_res: null pointer");
    if (((uintptr_t) C | (uintptr_t) h | (uintptr_t) sq) & 3)
        return fail(EXL3_AMD_EINVAL, "exl3_gemm_res: C, h and sq must be 4-byte aligned");
    DeviceState* d;
    if (int rc = current_device(&d, stream)) return rc;
    hipStream_t s = (hipStream_t) stream;
    if (m == 1)
    {
        // the residual add and the chunk sums in the epilogue of whichever GEMV kernel the plan
        // picks (the fused SwiGLU input needs the stream kernel)
        GemvArgs g = gemv_args_single(A, trellis, C, 0, suh, svh, m, k, n);
        GemvArgs probe = g;
        if (!gemv_plan(m, k, n, 1, d->num_cus, probe, WS_PARTIAL_BYTES) && (!up || probe.stream_m1 == 1))
        {
            g.A_up = up;
            g.res_h = h; g.res_sq = sq;
            int rc = launch_gemv(ws_of(d), bits, cb, g, s, "exl3_gemm_res");
            return rc ? rc : EXL3_AMD_TAG_GEMV;
        }
    }
    int tag = up ? exl3_amd_gemm_silu_mul(A, up, act, trellis, C, 0, suh, A_had, svh, m, k, n, K, mcg, mul1, stream)
                 : exl3_amd_gemm(A, trellis, C, 0, suh, A_had, svh, m, k, n, K, mcg, mul1, 0, stream);
    if (tag < 0) return tag;
    if (int rc = exl3k_res_sq(h, C, sq, m, n, s)) return hip_fail(rc, "exl3_gemm_res");
    return tag;
}

int exl3_amd_res_sq(uint16_t* h, const uint16_t* c, float* sq, int rows, int n, void* stream)
{
    g_last_error.clear();
    if (rows < 0 || n < 0) return fail(EXL3_AMD_EINVAL, "res_sq: negative size");
    if (n % 128) return fail(EXL3_AMD_EINVAL, "res_sq: n (%d) must be a multiple of 128", n);
    if (rows == 0 || n == 0) return 0;
    if (!h || !sq) return fail(EXL3_AMD_EINVAL, "res_sq: null pointer");
    if (((uintptr_t) h | (uintptr_t) c | (uintptr_t) sq) & 3) return fail(EXL3_AMD_EINVAL, "res_sq: pointers must be 4-byte aligned");
    if (rows > 65535) return fail(EXL3_AMD_EINVAL, "res_sq: at most 65535 rows");
    int rc = exl3k_res_sq(h, c, sq, rows, n, (hipStream_t) stream);
    return rc ? hip_fail(rc, "res_sq") : 0;
}

int exl3_amd_norm_sq(const uint16_t* h, const float* sq, const uint16_t* w, uint16_t* r, int rows, int n, float eps,
                     void* stream)
{
    g_last_error.clear();
    if (rows < 0 || n < 0) return fail(EXL3_AMD_EINVAL, "norm_sq: negative size");
    if (n % 128) return fail(EXL3_AMD_EINVAL, "norm_sq: n (%d) must be a multiple of 128", n);
    if (n > 64 * SQ_SCALE_MAX_PER_LANE * 128) return fail(EXL3_AMD_EINVAL, "norm_sq: n (%d) above %d", n, 64 * SQ_SCALE_MAX_PER_LANE * 128);
    if (rows == 0 || n == 0) return 0;
    if (!h || !sq || !w || !r) return fail(EXL3_AMD_EINVAL, "norm_sq: null pointer");
    if (((uintptr_t) h | (uintptr_t) sq | (uintptr_t) w | (uintptr_t) r) & 3)
        return fail(EXL3_AMD_EINVAL, "norm_sq: pointers must be 4-byte aligned");
    if (rows > 65535) return fail(EXL3_AMD_EINVAL, "norm_sq: at most 65535 rows");
    int rc = exl3k_norm_sq(h, sq, w, r, rows, n, eps, (hipStream_t) stream);
    return rc ? hip_fail(rc, "norm_sq") : 0;
}

}  // extern "C"
