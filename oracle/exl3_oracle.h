/*
 * exl3_oracle.h -- CPU restatement of the EXL3 quantized-linear arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * kernels in ampstein_amd/csrc: only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it.  The product path never calls it.
 *
 * Every function cites the reference file:line it restates (paths relative
 * to the jow-/ampstein tree, vendor/exl3 = exllamav3 v1.5.3 @ d3739fd).
 * Values of type h16 are IEEE binary16 bit patterns.
 */
#ifndef EXL3_ORACLE_H
#define EXL3_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t h16;

/* ---- binary16 arithmetic, each result rounded once (RNE) from the exact value ---- */
h16    exl3o_h_from_f64(double x);          /* double -> half, RNE (exact input assumed) */
h16    exl3o_h_from_f32(float x);           /* float  -> half, RNE (__float2half_rn)     */
float  exl3o_h_to_f32(h16 h);
h16    exl3o_hadd(h16 a, h16 b);            /* __hadd  */
h16    exl3o_hsub(h16 a, h16 b);            /* __hsub  */
h16    exl3o_hmul(h16 a, h16 b);            /* __hmul  */
h16    exl3o_hfma(h16 a, h16 b, h16 c);     /* __hfma: a*b+c, one rounding */

/* ---- a1: bitrate validation (quant/bits_k.cuh:178-185) ----
 * returns 0 and sets *bits / *half for K in {1..8} or {1.5,2.5,3.5}, else -1 */
int exl3o_bits_from_K(float K, int* bits, int* half);
int exl3o_tile_u16(int bits, int half);     /* 16*K (+8 for half-integer K) */

/* ---- a2: procedural codebooks (quant/codebook.cuh:57-90) ----
 * cb 0 = 3INST, 1 = MCG, 2 = MUL1.  state is the 16-bit trellis window. */
h16 exl3o_decode(uint32_t state, int cb);

/* ---- a3: window of tile position t (quant/exl3_dq.cuh:15-31, :254-285) ----
 * tile = 16*K (+8) uint16 words of one 16x16 tile. */
uint32_t exl3o_state(const uint16_t* tile, int bits, int half, int t);

/* ---- a4: tile permutation (cpu/moe_mul1.cpp:124-139, reconstruct.cu:36-85) ----
 * perm[p] = r*16 + c, the element of the 16x16 tile that position p decodes to. */
void exl3o_tile_perm(uint16_t perm[256]);

/* ---- a4: reconstruct (quant/reconstruct.cu:14-98, :141-194) ----
 * W_hat (k, n) fp16 row-major in the Hadamard basis.  n_offset (multiple of 16,
 * in columns) and the output width n select a column slice of a packed tensor
 * whose full width is n_packed.  Returns 0 or -1 on bad arguments. */
int exl3o_reconstruct(h16* W, const uint16_t* trellis, int k, int n, int n_packed,
                      int n_offset, int bits, int half, int cb, int nthreads);

/* ---- a5: fused original-basis reconstruct (quant/reconstruct.cu:212-364, :431-490) ----
 * W = diag(suh) . H . W_hat . H . diag(svh) per 128x128 block, with the reference's
 * fp16 rounding points.  k, n multiples of 128. */
int exl3o_reconstruct_had(h16* W, const uint16_t* trellis, const h16* suh, const h16* svh,
                          int k, int n, int n_packed, int n_offset,
                          int bits, int half, int cb, int nthreads);

/* The transform step of exl3o_reconstruct_had on a caller-supplied fp16 W_hat (k, n),
 * row-major: the same per-block sequence, without the trellis decode.  It exists so that
 * tests can feed the rounding sequence inputs whose results have closed forms. */
int exl3o_had_transform(h16* W, const h16* W_hat, const h16* suh, const h16* svh,
                        int k, int n, int nthreads);

/* ---- a6/a7: Hadamard-128 (quant/hadamard_inner.cuh:93-281, hadamard.cu:125-210) ----
 * y[r, 128j..] = H128(x[r, 128j..] (*pre)) * scale/sqrt(128) (*post), cols % 128 == 0.
 * pre/post are fp16 vectors of length cols (or NULL).  In place allowed. */
void exl3o_had128_hf(const h16* x, h16* y, int rows, int cols,
                     const h16* pre, const h16* post, float scale);   /* half in/out */
void exl3o_had128_ff(const float* x, float* y, int rows, int cols,
                     const h16* pre, const h16* post, float scale);   /* float in/out */
void exl3o_had128_fh(const float* x, h16* y, int rows, int cols,
                     const h16* post, float scale);                   /* GEMM epilogue */
/* Exact fp32 natural-order butterfly on one 128-vector (no scaling). */
void exl3o_fwht128_f32(float* v);

/* ---- a8..a12: reference linear (exl3_gemv_kernel.cuh:208-225, :454-481;
 *      exl3_gemm_inner.cuh:606-633) ----
 * x (m, k) fp16; W_hat from the trellis; y (m, n) fp16 (y_fp32 = 0) or fp32.
 *   A_had = had_hf(x, pre = suh)                    (fp16)
 *   P     = A_had @ W_hat, accumulated in double
 *   y     = had(P, post = svh): the half-output form rounds P to fp16 and uses
 *           had_hf; the float form uses had_ff.
 * suh / svh may be NULL (no rotation on that side, as exl3_gemm allows). */
int exl3o_linear(const h16* x, const uint16_t* trellis, const h16* suh, const h16* svh,
                 void* y, int m, int k, int n, int bits, int half, int cb, int y_fp32,
                 int nthreads);

/* fp64 evaluation of the same product, no intermediate rounding after A_had:
 * y = (H(P) / sqrt(128)) * svh in double.  y64 (m, n). */
int exl3o_linear_f64(const h16* x, const uint16_t* trellis, const h16* suh, const h16* svh,
                     double* y64, int m, int k, int n, int bits, int half, int cb,
                     int nthreads);

/* Dense product y (m,n) fp32 = x (m,k) fp16 @ W (k,n) fp16, double accumulation,
 * then rounded to fp32.  Used for the original-basis (prefill) form. */
void exl3o_matmul_h(const h16* x, const h16* W, float* y, int m, int k, int n, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
