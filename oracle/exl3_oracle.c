/*
 * exl3_oracle.c -- CPU restatement of the EXL3 quantized-linear arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels (see header).
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off: every fp32 operation
 * below must round exactly once, as the reference kernels' do).
 *
 * Pinning (tests/test_oracle*.py):
 *   - binary16 rounding: against numpy's float64->float16 cast (independent RNE
 *     implementation) on exhaustive / random operand sets;
 *   - codebooks: known-answer values and exhaustive-distribution statistics;
 *   - window extraction: independent bit-string implementation in Python and, where
 *     /root/reference is present, the compiled reference decode_state_scalar;
 *   - tile permutation: compiled reference make_tc_perm + single-bit perturbation;
 *   - Hadamard fp32 butterfly: compiled reference hadamard_128_scalar (bit-exact),
 *     H.H = I, symmetry, scipy Sylvester matrix;
 *   - linear: fp64 brute force and linearity.
 */
#include "exl3_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* binary16 rounding from an exact value N * 2^e                              */
/* ------------------------------------------------------------------------- */

typedef __int128 i128;

static int msb128(unsigned __int128 v)
{
    int p = 0;
    uint64_t hi = (uint64_t)(v >> 64);
    if (hi) { p = 64; v = hi; }
    uint64_t lo = (uint64_t) v;
    return p + 63 - __builtin_clzll(lo);
}

/* Round |N| * 2^e (N != 0) to binary16, RNE, with the given sign. */
static h16 round_half(unsigned __int128 N, int e, int neg)
{
    uint16_t sign = neg ? 0x8000 : 0;
    if (N == 0) return sign;
    int p = msb128(N);
    int E = p + e;                        /* value in [2^E, 2^(E+1)) */
    int qe = E - 10;                      /* quantum exponent of a normal result */
    if (qe < -24) qe = -24;               /* subnormal quantum */
    int shift = qe - e;
    unsigned __int128 M;
    if (shift <= 0)
    {
        M = N << (-shift);
    }
    else if (shift > p + 1)
    {
        M = 0;                            /* N < 2^(p+1) < half a quantum: rounds to zero */
    }
    else
    {
        M = N >> shift;
        unsigned __int128 rem = N - (M << shift);
        unsigned __int128 half_q = ((unsigned __int128) 1) << (shift - 1);
        if (rem > half_q || (rem == half_q && (M & 1))) M += 1;
    }
    if (M >= 2048) { M >>= 1; qe += 1; }  /* carry out of the mantissa */
    if (M == 0) return sign;
    if (qe == -24 && M < 1024) return sign | (uint16_t) M;     /* subnormal */
    int Eb = qe + 10 + 15;
    if (Eb >= 31) return sign | 0x7c00;                         /* overflow -> inf */
    return sign | (uint16_t)(Eb << 10) | (uint16_t)(M - 1024);
}

/* Exact decomposition of a finite half: value = m * 2^-24, m signed (|m| < 2^40). */
static int64_t half_units(h16 h)
{
    int64_t m;
    int ex = (h >> 10) & 31;
    int64_t f = h & 1023;
    if (ex == 0) m = f;
    else m = (1024 + f) << (ex - 1);
    return (h & 0x8000) ? -m : m;
}

static int half_is_special(h16 h) { return ((h >> 10) & 31) == 31; }

static float half_to_float_bits(h16 h)
{
    int ex = (h >> 10) & 31;
    uint32_t f = h & 1023;
    uint32_t s = (uint32_t)(h & 0x8000) << 16;
    uint32_t bits;
    if (ex == 31) bits = s | 0x7f800000u | (f << 13);
    else if (ex == 0)
    {
        if (f == 0) bits = s;
        else
        {
            int sh = 0;
            while (!(f & 1024)) { f <<= 1; sh++; }
            f &= 1023;
            bits = s | ((uint32_t)(127 - 15 + 1 - sh) << 23) | (f << 13);
        }
    }
    else bits = s | ((uint32_t)(ex - 15 + 127) << 23) | (f << 13);
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

float exl3o_h_to_f32(h16 h) { return half_to_float_bits(h); }

h16 exl3o_h_from_f64(double x)
{
    if (isnan(x)) return 0x7e00;
    if (isinf(x)) return x < 0 ? 0xfc00 : 0x7c00;
    int neg = signbit(x) ? 1 : 0;
    double a = fabs(x);
    if (a == 0.0) return neg ? 0x8000 : 0;
    int ex;
    double m = frexp(a, &ex);             /* a = m * 2^ex, m in [0.5, 1) */
    uint64_t N = (uint64_t) ldexp(m, 53); /* exact */
    return round_half(N, ex - 53, neg);
}

h16 exl3o_h_from_f32(float x) { return exl3o_h_from_f64((double) x); }

/* Rounded results of exact sums/products; NaN/Inf operands propagate as in IEEE. */
static h16 special_result(double exact_via_float)
{
    return exl3o_h_from_f64(exact_via_float);
}

h16 exl3o_hadd(h16 a, h16 b)
{
    if (half_is_special(a) || half_is_special(b))
        return special_result((double) half_to_float_bits(a) + (double) half_to_float_bits(b));
    int64_t s = half_units(a) + half_units(b);
    if (s == 0)   /* RNE: exact zero sum is +0 unless both operands are -0 */
        return ((a & 0x8000) && (b & 0x8000)) ? 0x8000 : 0;
    return round_half((unsigned __int128)(s < 0 ? -s : s), -24, s < 0);
}

h16 exl3o_hsub(h16 a, h16 b) { return exl3o_hadd(a, b ^ 0x8000); }

h16 exl3o_hmul(h16 a, h16 b)
{
    if (half_is_special(a) || half_is_special(b))
        return special_result((double) half_to_float_bits(a) * (double) half_to_float_bits(b));
    i128 p = (i128) half_units(a) * (i128) half_units(b);
    int neg = ((a ^ b) & 0x8000) != 0;
    if (p == 0) return neg ? 0x8000 : 0;
    return round_half((unsigned __int128)(p < 0 ? -p : p), -48, p < 0);
}

h16 exl3o_hfma(h16 a, h16 b, h16 c)
{
    if (half_is_special(a) || half_is_special(b) || half_is_special(c))
        return special_result((double) half_to_float_bits(a) * (double) half_to_float_bits(b)
                              + (double) half_to_float_bits(c));
    i128 p = (i128) half_units(a) * (i128) half_units(b);
    i128 s = p + ((i128) half_units(c) << 24);
    if (s == 0)
    {
        int pneg = ((a ^ b) & 0x8000) != 0;
        return (pneg && (c & 0x8000)) ? 0x8000 : 0;
    }
    return round_half((unsigned __int128)(s < 0 ? -s : s), -48, s < 0);
}

/* ------------------------------------------------------------------------- */
/* a1: bitrate (quant/bits_k.cuh:178-185)                                     */
/* ------------------------------------------------------------------------- */

int exl3o_bits_from_K(float K, int* bits, int* half)
{
    int b = (int) K;
    float f = K - (float) b;
    if (!(b >= 1 && b <= 8 && (f == 0.0f || (f == 0.5f && b <= 3)))) return -1;
    if (bits) *bits = b;
    if (half) *half = f == 0.5f;
    return 0;
}

int exl3o_tile_u16(int bits, int half) { return 16 * bits + (half ? 8 : 0); }

/* ------------------------------------------------------------------------- */
/* a2: codebooks (quant/codebook.cuh:57-90)                                   */
/* ------------------------------------------------------------------------- */

h16 exl3o_decode(uint32_t state, int cb)
{
    uint32_t x = state & 0xffffu;
    if (cb == 0 || cb == 1)
    {
        if (cb == 0) x = x * 89226354u + 64248484u;      /* codebook.cuh:61-62 */
        else         x = x * 0xCBAC1FEDu;                /* codebook.cuh:69    */
        x = (x & 0x8fff8fffu) ^ 0x3b603b60u;             /* lop3 0x6a: (a & b) ^ c */
        return exl3o_hadd((h16)(x & 0xffff), (h16)(x >> 16));
    }
    /* cb == 2, mul1 (codebook.cuh:78-88): byte sum + 0x6400 as an fp16 in [1024, 2047],
       then one fp16 fma with k_inv = 0x1eee and bias = 0xc931 */
    x = x * 0x83DCD12Du;
    uint32_t sum = (x & 0xff) + ((x >> 8) & 0xff) + ((x >> 16) & 0xff) + (x >> 24) + 0x6400u;
    return exl3o_hfma((h16) sum, (h16) 0x1eee, (h16) 0xc931);
}

/* ------------------------------------------------------------------------- */
/* a3: window extraction (quant/exl3_dq.cuh:15-31 integer K, :254-285 half K)  */
/* ------------------------------------------------------------------------- */

static inline uint32_t tile_word(const uint16_t* tile, int i)
{
    return (uint32_t) tile[2 * i] | ((uint32_t) tile[2 * i + 1] << 16);
}

/* End bit (exclusive, MSB-first numbering, one ring ahead) of position t's window. */
static inline int window_end(int bits, int half, int t)
{
    if (!half) return t * bits + bits + 256 * bits;                  /* exl3_dq.cuh:18-19 */
    int bits2 = 2 * bits + 1;                                        /* even t: bits, odd t: bits+1 */
    return (t >> 1) * bits2 + ((t & 1) ? bits2 : bits) + 128 * bits2;
}

uint32_t exl3o_state(const uint16_t* tile, int bits, int half, int t)
{
    int words = exl3o_tile_u16(bits, half) / 2;
    int e = window_end(bits, half, t);
    int ihi = (e - 1) / 32;                 /* word holding the window's last bit  */
    int ilo = (e - 16) / 32;                /* word holding the window's first bit */
    int s = (ihi + 1) * 32 - e;             /* right shift aligning the last bit to bit 0 */
    uint64_t merged = ((uint64_t) tile_word(tile, ilo % words) << 32) | tile_word(tile, ihi % words);
    return (uint32_t)(merged >> s) & 0xffffu;
}

/* ------------------------------------------------------------------------- */
/* a4: tile permutation + reconstruct                                          */
/* ------------------------------------------------------------------------- */

void exl3o_tile_perm(uint16_t perm[256])
{
    /* Lane L of a 32-lane group decodes positions 8L..8L+7 (reconstruct.cu:37-38); the
       shuffle at reconstruct.cu:44-84 lands them at rows r0, r0+1, r0+8, r0+9 of column
       L/4 (j = 0..3) and column L/4 + 8 (j = 4..7), r0 = 2 (L % 4). */
    for (int L = 0; L < 32; ++L)
    {
        int r0 = (L % 4) * 2;
        int c0 = L / 4;
        static const int dr[4] = { 0, 1, 8, 9 };
        for (int j = 0; j < 8; ++j)
        {
            int r = r0 + dr[j & 3];
            int c = c0 + (j >= 4 ? 8 : 0);
            perm[8 * L + j] = (uint16_t)(r * 16 + c);
        }
    }
}

typedef void (*range_fn)(void* ctx, int begin, int end);
struct job { range_fn fn; void* ctx; int begin, end; };

static void* job_run(void* p)
{
    struct job* j = (struct job*) p;
    j->fn(j->ctx, j->begin, j->end);
    return NULL;
}

static void parallel_for(range_fn fn, void* ctx, int count, int nthreads)
{
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 64) nthreads = 64;
    if (nthreads > count) nthreads = count > 0 ? count : 1;
    if (nthreads == 1) { fn(ctx, 0, count); return; }
    pthread_t th[64];
    struct job jobs[64];
    int per = (count + nthreads - 1) / nthreads;
    int started = 0;
    for (int i = 0; i < nthreads; ++i)
    {
        int b = i * per, e = b + per;
        if (e > count) e = count;
        if (b >= e) break;
        jobs[i] = (struct job){ fn, ctx, b, e };
        if (pthread_create(&th[i], NULL, job_run, &jobs[i]) != 0) { job_run(&jobs[i]); th[i] = 0; }
        started = i + 1;
    }
    for (int i = 0; i < started; ++i) if (th[i]) pthread_join(th[i], NULL);
}

struct recon_ctx
{
    h16* W; const uint16_t* trellis; int k, n, n_packed, n_offset, bits, half, cb;
    uint16_t perm[256];
};

static void decode_tile(h16 out[256], const uint16_t* tile, int bits, int half, int cb,
                        const uint16_t* perm)
{
    for (int p = 0; p < 256; ++p)
        out[perm[p]] = exl3o_decode(exl3o_state(tile, bits, half, p), cb);
}

static void recon_rows(void* vctx, int kt0, int kt1)
{
    struct recon_ctx* c = (struct recon_ctx*) vctx;
    int tu16 = exl3o_tile_u16(c->bits, c->half);
    int tiles_n = c->n_packed / 16;
    h16 tile[256];
    for (int kt = kt0; kt < kt1; ++kt)
        for (int j = 0; j < c->n / 16; ++j)
        {
            int nt = c->n_offset / 16 + j;
            const uint16_t* tp = c->trellis + ((size_t) kt * tiles_n + nt) * tu16;
            decode_tile(tile, tp, c->bits, c->half, c->cb, c->perm);
            for (int r = 0; r < 16; ++r)
                memcpy(c->W + (size_t)(kt * 16 + r) * c->n + j * 16, tile + r * 16, 32);
        }
}

int exl3o_reconstruct(h16* W, const uint16_t* trellis, int k, int n, int n_packed,
                      int n_offset, int bits, int half, int cb, int nthreads)
{
    if (k % 16 || n % 16 || n_offset % 16 || n_offset < 0 || n_offset + n > n_packed) return -1;
    if (bits < 1 || bits > 8 || (half && (bits > 3 || cb != 2)) || cb < 0 || cb > 2) return -1;
    struct recon_ctx c = { W, trellis, k, n, n_packed, n_offset, bits, half, cb, {0} };
    exl3o_tile_perm(c.perm);
    parallel_for(recon_rows, &c, k / 16, nthreads);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* a6/a7: Hadamard-128                                                        */
/* ------------------------------------------------------------------------- */

void exl3o_fwht128_f32(float* v)
{
    /* Element 4t+i lives in lane t: the in-lane 4-point stage (widths 1, 2) and the
       xor-1..16 lane stages (widths 4..64) of hadamard_inner.cuh:17-41, :119-134 are the
       natural-order in-place butterfly below, lower index a+b, upper a-b. */
    for (int w = 1; w < 128; w <<= 1)
        for (int base = 0; base < 128; base += 2 * w)
            for (int i = 0; i < w; ++i)
            {
                float a = v[base + i], b = v[base + w + i];
                v[base + i] = a + b;
                v[base + w + i] = a - b;
            }
}

void exl3o_had128_hf(const h16* x, h16* y, int rows, int cols,
                     const h16* pre, const h16* post, float scale)
{
    /* hadamard.cu:166 computes r_scale in float; hadamard_inner.cuh:93-150 */
    const float r_scale = scale * 0.088388347648f;
    float v[128];
    for (int r = 0; r < rows; ++r)
        for (int c0 = 0; c0 < cols; c0 += 128)
        {
            const h16* xi = x + (size_t) r * cols + c0;
            for (int i = 0; i < 128; ++i)
            {
                h16 h = xi[i];
                if (pre) h = exl3o_hmul(h, pre[c0 + i]);
                v[i] = half_to_float_bits(h);
            }
            exl3o_fwht128_f32(v);
            h16* yo = y + (size_t) r * cols + c0;
            for (int i = 0; i < 128; ++i)
            {
                h16 h = exl3o_h_from_f32(v[i] * r_scale);
                if (post) h = exl3o_hmul(h, post[c0 + i]);
                yo[i] = h;
            }
        }
}

void exl3o_had128_ff(const float* x, float* y, int rows, int cols,
                     const h16* pre, const h16* post, float scale)
{
    /* hadamard_inner.cuh:154-211 */
    const float r_scale = scale * 0.088388347648f;
    float v[128];
    for (int r = 0; r < rows; ++r)
        for (int c0 = 0; c0 < cols; c0 += 128)
        {
            const float* xi = x + (size_t) r * cols + c0;
            for (int i = 0; i < 128; ++i)
                v[i] = pre ? xi[i] * half_to_float_bits(pre[c0 + i]) : xi[i];
            exl3o_fwht128_f32(v);
            float* yo = y + (size_t) r * cols + c0;
            for (int i = 0; i < 128; ++i)
            {
                float t = v[i] * r_scale;
                yo[i] = post ? t * half_to_float_bits(post[c0 + i]) : t;
            }
        }
}

void exl3o_had128_fh(const float* x, h16* y, int rows, int cols, const h16* post, float scale)
{
    /* hadamard_inner.cuh:216-281 */
    const float r_scale = scale * 0.088388347648f;
    float v[128];
    for (int r = 0; r < rows; ++r)
        for (int c0 = 0; c0 < cols; c0 += 128)
        {
            memcpy(v, x + (size_t) r * cols + c0, sizeof(v));
            exl3o_fwht128_f32(v);
            h16* yo = y + (size_t) r * cols + c0;
            for (int i = 0; i < 128; ++i)
            {
                h16 h = exl3o_h_from_f32(v[i] * r_scale);
                yo[i] = post ? exl3o_hmul(h, post[c0 + i]) : h;
            }
        }
}

/* ------------------------------------------------------------------------- */
/* a5: fused original-basis reconstruct (quant/reconstruct.cu:212-364)         */
/* ------------------------------------------------------------------------- */

/* fp16 natural-order butterfly over 128 values with the lane split of
   reconstruct.cu:290-318 (column pass) / :331-357 (row pass):
   in-lane 4-point stage, times rs, then shuffle_had_h2x32 (hadamard_inner.cuh:83-93). */
static void had128_h16_lane_stages(h16* v)
{
    /* lane stages: element 4t+i, partner lane t^s -> element distance 4s */
    for (int w = 4; w < 128; w <<= 1)
        for (int base = 0; base < 128; base += 2 * w)
            for (int i = 0; i < w; ++i)
            {
                h16 a = v[base + i], b = v[base + w + i];
                v[base + i] = exl3o_hadd(a, b);            /* lower lane: v + pv          */
                v[base + w + i] = exl3o_hadd(b ^ 0x8000, a); /* upper lane: (-v) + pv     */
            }
}

/* The two-pass Hadamard of one 128 x 128 block, in place in blk (row-major, stride 128), then
   out[R * out_stride + C] = result * su[R] * sv[C] (reconstruct.cu:290-357). */
static void had_block_h16(h16* blk, const h16* su, const h16* sv, h16* out, size_t out_stride)
{
    const h16 rs = exl3o_h_from_f32(0.08838834764831845f);   /* __float2half2_rn(r_scale) */
    h16 v[128];
    /* column pass (reconstruct.cu:290-318): per column, over the 128 rows; fp16 4-point
       stage, each result times rs, then fp16 lane stages */
    for (int col = 0; col < 128; ++col)
    {
        for (int R = 0; R < 128; ++R) v[R] = blk[R * 128 + col];
        for (int t = 0; t < 32; ++t)
        {
            h16* q = v + 4 * t;
            h16 s0 = exl3o_hadd(q[0], q[1]), d0 = exl3o_hsub(q[0], q[1]);
            h16 s1 = exl3o_hadd(q[2], q[3]), d1 = exl3o_hsub(q[2], q[3]);
            q[0] = exl3o_hmul(exl3o_hadd(s0, s1), rs);
            q[1] = exl3o_hmul(exl3o_hadd(d0, d1), rs);
            q[2] = exl3o_hmul(exl3o_hsub(s0, s1), rs);
            q[3] = exl3o_hmul(exl3o_hsub(d0, d1), rs);
        }
        had128_h16_lane_stages(v);
        for (int R = 0; R < 128; ++R) blk[R * 128 + col] = v[R];
    }
    /* row pass fused with the store (reconstruct.cu:331-357): fp32 4-point stage,
       round to half, times rs in fp16, fp16 lane stages, then * su[row] * sv[col] */
    for (int R = 0; R < 128; ++R)
    {
        h16* row = blk + R * 128;
        for (int t = 0; t < 32; ++t)
        {
            float v0 = half_to_float_bits(row[4 * t + 0]);
            float v1 = half_to_float_bits(row[4 * t + 1]);
            float v2 = half_to_float_bits(row[4 * t + 2]);
            float v3 = half_to_float_bits(row[4 * t + 3]);
            float s0 = v0 + v1, d0 = v0 - v1, s1 = v2 + v3, d1 = v2 - v3;
            v[4 * t + 0] = exl3o_hmul(exl3o_h_from_f32(s0 + s1), rs);
            v[4 * t + 1] = exl3o_hmul(exl3o_h_from_f32(d0 + d1), rs);
            v[4 * t + 2] = exl3o_hmul(exl3o_h_from_f32(s0 - s1), rs);
            v[4 * t + 3] = exl3o_hmul(exl3o_h_from_f32(d0 - d1), rs);
        }
        had128_h16_lane_stages(v);
        h16* o = out + (size_t) R * out_stride;
        for (int i = 0; i < 128; ++i)
            o[i] = exl3o_hmul(exl3o_hmul(v[i], su[R]), sv[i]);
    }
}

struct rh_ctx
{
    h16* W; const uint16_t* trellis; const h16* W_hat; const h16* suh; const h16* svh;
    int k, n, n_packed, n_offset, bits, half, cb;
    uint16_t perm[256];
};

static void rh_blocks(void* vctx, int b0, int b1)
{
    struct rh_ctx* c = (struct rh_ctx*) vctx;
    const int tu16 = c->W_hat ? 0 : exl3o_tile_u16(c->bits, c->half);
    const int tiles_n = c->n_packed / 16;
    const int nblk = c->n / 128;
    h16* blk = (h16*) malloc(128 * 128 * sizeof(h16));
    h16 tile[256];
    for (int b = b0; b < b1; ++b)
    {
        int kb = b / nblk, nb = b % nblk;
        if (c->W_hat)
        {
            /* caller-supplied W_hat (k x n, row-major) */
            for (int R = 0; R < 128; ++R)
                memcpy(blk + R * 128, c->W_hat + (size_t)(kb * 128 + R) * c->n + nb * 128, 256);
        }
        else
        {
            /* decode 8x8 tiles into the 128x128 block (rows = k, cols = n) */
            for (int j = 0; j < 8; ++j)
                for (int wn = 0; wn < 8; ++wn)
                {
                    int nt = c->n_offset / 16 + nb * 8 + wn;
                    const uint16_t* tp = c->trellis + ((size_t)(kb * 8 + j) * tiles_n + nt) * tu16;
                    decode_tile(tile, tp, c->bits, c->half, c->cb, c->perm);
                    for (int r = 0; r < 16; ++r)
                        memcpy(blk + (j * 16 + r) * 128 + wn * 16, tile + r * 16, 32);
                }
        }
        had_block_h16(blk, c->suh + kb * 128, c->svh + nb * 128,
                      c->W + (size_t)(kb * 128) * c->n + nb * 128, (size_t) c->n);
    }
    free(blk);
}

int exl3o_reconstruct_had(h16* W, const uint16_t* trellis, const h16* suh, const h16* svh,
                          int k, int n, int n_packed, int n_offset,
                          int bits, int half, int cb, int nthreads)
{
    if (k % 128 || n % 128 || n_offset % 128 || n_offset < 0 || n_offset + n > n_packed) return -1;
    if (bits < 1 || bits > 8 || (half && (bits > 3 || cb != 2)) || cb < 0 || cb > 2) return -1;
    struct rh_ctx c = { W, trellis, NULL, suh, svh, k, n, n_packed, n_offset, bits, half, cb, {0} };
    exl3o_tile_perm(c.perm);
    parallel_for(rh_blocks, &c, (k / 128) * (n / 128), nthreads);
    return 0;
}

int exl3o_had_transform(h16* W, const h16* W_hat, const h16* suh, const h16* svh,
                        int k, int n, int nthreads)
{
    if (k % 128 || n % 128 || k <= 0 || n <= 0) return -1;
    struct rh_ctx c = { W, NULL, W_hat, suh, svh, k, n, n, 0, 0, 0, 0, {0} };
    parallel_for(rh_blocks, &c, (k / 128) * (n / 128), nthreads);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* Reference linear                                                            */
/* ------------------------------------------------------------------------- */

struct mm_ctx { const h16* A; const h16* W; double* P; int m, k, n; };

static void mm_cols(void* vctx, int c0, int c1)
{
    /* P[:, 64-column blocks c0 .. c1) = A @ W in double, W row-major (k, n) */
    struct mm_ctx* c = (struct mm_ctx*) vctx;
    double wrow[64];
    for (int blk = c0; blk < c1; ++blk)
    {
        int j0 = blk * 64, j1 = j0 + 64;
        if (j1 > c->n) j1 = c->n;
        for (int r = 0; r < c->m; ++r)
        {
            double* pr = c->P + (size_t) r * c->n;
            for (int j = j0; j < j1; ++j) pr[j] = 0.0;
            for (int i = 0; i < c->k; ++i)
            {
                double a = half_to_float_bits(c->A[(size_t) r * c->k + i]);
                if (a == 0.0) continue;
                const h16* wr = c->W + (size_t) i * c->n;
                for (int j = j0; j < j1; ++j) wrow[j - j0] = half_to_float_bits(wr[j]);
                for (int j = j0; j < j1; ++j) pr[j] += a * wrow[j - j0];
            }
        }
    }
}

static void matmul_d(const h16* A, const h16* W, double* P, int m, int k, int n, int nthreads)
{
    struct mm_ctx c = { A, W, P, m, k, n };
    parallel_for(mm_cols, &c, (n + 63) / 64, nthreads);
}

void exl3o_matmul_h(const h16* x, const h16* W, float* y, int m, int k, int n, int nthreads)
{
    double* P = (double*) malloc(sizeof(double) * (size_t) m * n);
    matmul_d(x, W, P, m, k, n, nthreads);
    for (size_t i = 0; i < (size_t) m * n; ++i) y[i] = (float) P[i];
    free(P);
}

static int linear_common(const h16* x, const uint16_t* trellis, const h16* suh,
                         int m, int k, int n, int bits, int half, int cb, int nthreads,
                         double** P_out)
{
    if (k % 128 || n % 128 || m < 0) return -1;
    h16* W = (h16*) malloc(sizeof(h16) * (size_t) k * n);
    h16* A = (h16*) malloc(sizeof(h16) * (size_t) m * k + 2);
    double* P = (double*) malloc(sizeof(double) * (size_t) m * n + 8);
    if (exl3o_reconstruct(W, trellis, k, n, n, 0, bits, half, cb, nthreads)) { free(W); free(A); free(P); return -1; }
    if (suh) exl3o_had128_hf(x, A, m, k, suh, NULL, 1.0f);
    else memcpy(A, x, sizeof(h16) * (size_t) m * k);
    matmul_d(A, W, P, m, k, n, nthreads);
    free(W); free(A);
    *P_out = P;
    return 0;
}

int exl3o_linear(const h16* x, const uint16_t* trellis, const h16* suh, const h16* svh,
                 void* y, int m, int k, int n, int bits, int half, int cb, int y_fp32,
                 int nthreads)
{
    double* P;
    if (linear_common(x, trellis, suh, m, k, n, bits, half, cb, nthreads, &P)) return -1;
    size_t mn = (size_t) m * n;
    if (y_fp32)
    {
        float* yf = (float*) y;
        for (size_t i = 0; i < mn; ++i) yf[i] = (float) P[i];
        if (svh) exl3o_had128_ff(yf, yf, m, n, NULL, svh, 1.0f);
    }
    else
    {
        h16* yh = (h16*) y;
        for (size_t i = 0; i < mn; ++i) yh[i] = exl3o_h_from_f64(P[i]);
        if (svh) exl3o_had128_hf(yh, yh, m, n, NULL, svh, 1.0f);
    }
    free(P);
    return 0;
}

int exl3o_linear_f64(const h16* x, const uint16_t* trellis, const h16* suh, const h16* svh,
                     double* y64, int m, int k, int n, int bits, int half, int cb, int nthreads)
{
    double* P;
    if (linear_common(x, trellis, suh, m, k, n, bits, half, cb, nthreads, &P)) return -1;
    const double rs = 1.0 / sqrt(128.0);
    double v[128];
    for (int r = 0; r < m; ++r)
        for (int c0 = 0; c0 < n; c0 += 128)
        {
            memcpy(v, P + (size_t) r * n + c0, sizeof(v));
            if (svh)
                for (int w = 1; w < 128; w <<= 1)
                    for (int base = 0; base < 128; base += 2 * w)
                        for (int i = 0; i < w; ++i)
                        {
                            double a = v[base + i], b = v[base + w + i];
                            v[base + i] = a + b;
                            v[base + w + i] = a - b;
                        }
            for (int i = 0; i < 128; ++i)
                y64[(size_t) r * n + c0 + i] = svh ? v[i] * rs * half_to_float_bits(svh[c0 + i]) : v[i];
        }
    free(P);
    return 0;
}
