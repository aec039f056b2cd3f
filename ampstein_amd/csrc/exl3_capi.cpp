// C-ABI entry points of libexl3_amd.so (declared in include/exl3_amd.h).
//
// Every argument check of the reference's TORCH_CHECKs for these operators is made here,
// before any launch, and reported as an error code plus a thread-local message instead of
// an exception (quant/reconstruct.cu:152-176, hadamard.cu:141-145, exl3_gemm.cu:128-176,
// bits_k.cuh:178-185).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
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
// both_ok: the reconstruct entry points take mcg over mul1 when both are set
// (reconstruct.cu:181-184); exl3_gemm rejects the combination (exl3_gemm.cu:179).
int parse_K(float K, int mcg, int mul1, int* bits, int* half, int* cb, const char* what, bool both_ok = false)
{
    const int b = (int) K;
    const float f = K - (float) b;
    if (!(b >= 1 && b <= 8 && (f == 0.0f || (f == 0.5f && b <= 3))))
        return fail(EXL3_AMD_EINVAL, "%s: unsupported EXL3 bitrate %g (integer 1..8, or 1.5 / 2.5 / 3.5)", what, (double) K);
    if (mcg && mul1 && !both_ok) return fail(EXL3_AMD_EINVAL, "%s: specified both mcg and mul1", what);
    *bits = b;
    *half = f == 0.5f;
    *cb = mcg ? 1 : (mul1 ? 2 : 0);
    if (*half && mul1) *cb = 2;
    if (*half && !mul1) return fail(EXL3_AMD_EINVAL, "%s: half-integer bitrates require the mul1 codebook", what);
    if (*half) return fail(EXL3_AMD_EUNSUPPORTED, "%s: half-integer bitrates are not implemented in this build", what);
    return 0;
}

// ------------------------------------------------------------------ per-device workspace
constexpr int MAX_DEVICES = 16;
constexpr size_t WS_PARTIAL_BYTES = 64ull << 20;     // split-k fp32 partials
constexpr size_t WS_COUNTERS = 1u << 20;             // column-chunk completion counters

struct DeviceState
{
    bool ready = false;
    int num_cus = 0;
    int num_xcd = 0;            // > 0 when workgroup b is verified to run on XCD b % num_xcd
    float* partials = nullptr;
    int* counters = nullptr;
};

DeviceState g_dev[MAX_DEVICES];
std::mutex g_mutex;

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
            if (hipMalloc(&c, WS_COUNTERS * sizeof(int)) != hipSuccess)
            {
                (void) hipFree(p);
                return fail(EXL3_AMD_ENOMEM, "counter allocation failed");
            }
            if (hipMemset(c, 0, WS_COUNTERS * sizeof(int)) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
                return fail(EXL3_AMD_EHIP, "counter initialisation failed");
            // workgroup -> XCD dispatch order (round-robin on MI355X), verified on this device
            {
                const int sizes[3] = { 64, 1000, 8192 };
                int* probe = (int*) p;
                int nx = 0;
                bool ok = true;
                for (int si = 0; si < 3 && ok; ++si)
                {
                    int* host = (int*) malloc(sizes[si] * sizeof(int));
                    if (!host || exl3k_xcd_probe(probe, sizes[si], nullptr) || hipDeviceSynchronize() != hipSuccess ||
                        hipMemcpy(host, probe, sizes[si] * sizeof(int), hipMemcpyDeviceToHost) != hipSuccess)
                        ok = false;
                    if (ok)
                    {
                        int mx = 0;
                        for (int i = 0; i < sizes[si]; ++i) mx = host[i] > mx ? host[i] : mx;
                        if (si == 0) nx = mx + 1;
                        for (int i = 0; i < sizes[si] && ok; ++i) ok = host[i] == i % nx;
                    }
                    free(host);
                }
                d.num_xcd = ok && nx >= 1 ? nx : 0;
                if (const char* e = getenv("EXL3_AMD_XCD")) if (atoi(e) == 0) d.num_xcd = 0;
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

int current_device(DeviceState** out)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(EXL3_AMD_EHIP, "hipGetDevice failed");
    return init_device(dev, out);
}

// GEMV work split (exl3_gemv.hip): SB slices per workgroup, a divisor of k/16 (so no
// workgroup straddles two column chunks), sized for ~TARGET workgroups per CU within the LDS
// budget (rotated input + reduction buffer) and the split-partial workspace.
int gemv_plan(int m, int k, int n, int num_cus, GemvArgs& g)
{
    const int mt = m == 1 ? 1 : (m <= 4 ? 4 : 8);
    const int KS = k / 16, chunks = n / 128;
    int per_cu = 2;
    if (const char* e = getenv("EXL3_AMD_GEMV_WG_PER_CU")) { int v = atoi(e); if (v > 0) per_cu = v; }
    const long target = (long) per_cu * num_cus;
    // M = 1 streaming kernel: whole 128-row input chunks per wave (SB multiple of 32)
    int stream = m == 1 && KS % 32 == 0;
    if (const char* e = getenv("EXL3_AMD_GEMV_STREAM")) stream = stream && atoi(e) != 0;
    const int step = stream ? 32 : 1;
    const int lds_budget = 64 * 1024 - 4 * mt * 128 * 4;
    const int max_chunks = lds_budget / (mt * 512);           // rotated 128-row chunks in LDS
    int best = -1;
    for (int d = step; d <= KS; d += step)
    {
        if (KS % d) continue;
        if (!stream && d / 8 + 2 > max_chunks) break;
        if ((size_t) (KS / d) * m * n * 4 > WS_PARTIAL_BYTES && KS / d > 1) continue;
        if (best < 0 || (long) chunks * (KS / best) > target) best = d;   // fewest blocks >= target
        if ((long) chunks * (KS / d) <= target) break;
    }
    if (const char* e = getenv("EXL3_AMD_GEMV_SB")) { int v = atoi(e); if (v > 0 && KS % v == 0 && v % step == 0) best = v; }
    if (best < 0) return -1;
    g.stream_m1 = stream;
    g.slices_per_block = best;
    g.slots = KS / best;
    g.xs_chunks = best / 8 + 2;
    return 0;
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
    }
    return -1;
}

}  // namespace

extern "C" {

const char* exl3_amd_last_error(void) { return g_last_error.c_str(); }

int exl3_amd_version(void) { return 100; }

int exl3_amd_init(int device)
{
    DeviceState* d;
    return init_device(device, &d);
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

int exl3_amd_had_r_128(const void* x, void* y, int rows, int cols, int fp32,
                       const uint16_t* pre, const uint16_t* post, float scale, void* stream)
{
    g_last_error.clear();
    if (rows < 0 || cols < 0) return fail(EXL3_AMD_EINVAL, "had_r_128: negative size");
    if (cols % 128) return fail(EXL3_AMD_EINVAL, "had_r_128: columns must be divisible by 128");
    if (pre && post) return fail(EXL3_AMD_EINVAL, "had_r_128: give pre or post scale, not both");
    if ((size_t) rows * cols == 0) return 0;
    if (!x || !y) return fail(EXL3_AMD_EINVAL, "had_r_128: null pointer");
    int rc = exl3k_had128(x, y, rows, cols, fp32 ? 1 : 0, pre, post, scale, (hipStream_t) stream);
    return rc ? hip_fail(rc, "had_r_128") : 0;
}

int exl3_amd_gemm(const uint16_t* A, const uint16_t* trellis, void* C, int c_fp32,
                  const uint16_t* suh, uint16_t* A_had, const uint16_t* svh,
                  int m, int k, int n, float K, int mcg, int mul1, int force_shape_idx,
                  void* stream)
{
    (void) A_had;
    g_last_error.clear();
    int bits, half, cb;
    if (int rc = parse_K(K, mcg, mul1, &bits, &half, &cb, "exl3_gemm")) return rc;
    if (m < 0 || k < 0 || n < 0) return fail(EXL3_AMD_EINVAL, "exl3_gemm: negative size");
    if (k % 16) return fail(EXL3_AMD_EINVAL, "exl3_gemm: k must be a multiple of 16");
    if (n % 128) return fail(EXL3_AMD_EINVAL, "exl3_gemm: n must be a multiple of 128");
    if (m == 0 || n == 0) return EXL3_AMD_TAG_GEMV;
    if (!A || !trellis || !C) return fail(EXL3_AMD_EINVAL, "exl3_gemm: null pointer");
    if (k == 0) return fail(EXL3_AMD_EINVAL, "exl3_gemm: k must be positive");
    if (k % 128) return fail(EXL3_AMD_EUNSUPPORTED, "exl3_gemm: k %% 128 != 0 is not implemented in this build");
    if (force_shape_idx < 0 || force_shape_idx > 2) return fail(EXL3_AMD_EINVAL, "exl3_gemm: bad force_shape_idx %d", force_shape_idx);

    DeviceState* d;
    if (int rc = current_device(&d)) return rc;
    hipStream_t s = (hipStream_t) stream;

    if (m <= 8 && force_shape_idx != 2)
    {
        GemvArgs g;
        g.A = A; g.trellis = trellis; g.C = C; g.suh = suh; g.svh = svh;
        g.m = m; g.k = k; g.n = n; g.c_fp32 = c_fp32 ? 1 : 0;
        if (gemv_plan(m, k, n, d->num_cus, g)) return fail(EXL3_AMD_EUNSUPPORTED, "exl3_gemm: shape exceeds the GEMV workspace");
        g.partials = d->partials;
        g.counters = d->counters;
        g.xcd = 0;
        if (g.stream_m1 && d->num_xcd > 0 && (n / 128) % d->num_xcd == 0 && (size_t) (n / 128) * 32 <= WS_COUNTERS)
            g.xcd = d->num_xcd;
        if ((size_t) n / 128 > WS_COUNTERS) return fail(EXL3_AMD_EUNSUPPORTED, "exl3_gemm: n too large for the counter workspace");
        int rc = dispatch_gemv(bits, cb, g, s);
        return rc ? hip_fail(rc, "exl3_gemm") : EXL3_AMD_TAG_GEMV;
    }
    return fail(EXL3_AMD_EUNSUPPORTED, "exl3_gemm: m > 8 (MFMA GEMM) is not implemented in this build");
}

}  // extern "C"
