/*
 * oracle/sam3_oracle.h - CPU restatement of sam3.c's matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the
 * HIP backend and the timed CPU baseline ("port") of bench.py. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it; the product path (sam3.c_amd) never links or calls it.
 *
 * Every function restates one reference routine with the same
 * per-element arithmetic order, so that results are bit-identical to
 * the reference compiled as its x86 scalar build (-std=c11 -O2, no
 * -march, no BLAS, no FP contraction). Reference citations are given as
 * /root/reference/<path>:<line>.
 *
 * Pinning (tests/test_oracle.py): golden vectors written by the real
 * reference (tests/golden/), a direct comparison against
 * oracle/_ref/libsam3ref.so when it is built, the reference tests' own
 * known answers, exhaustive conversion sweeps, and closed forms
 * (identity, one-hot rows, float64 brute force).
 */
#ifndef SAM3_ORACLE_H
#define SAM3_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#define ORACLE_Q8_BLOCK 32
#define ORACLE_Q8_BLOCK_BYTES 36

/* ---- Q8_0 format (src/core/quant.h:22-33, src/core/quant.c:29-165) ---- */
int    oracle_q8_block_count(int nelems);
size_t oracle_q8_nbytes(int nelems);
void   oracle_q8_quantize(const float *src, void *dst_blocks, int nelems);
void   oracle_q8_dequantize(const void *src_blocks, float *dst, int nelems);

/* ---- fp16 / bf16 scalar conversions (src/core/half.h:58-210) ---- */
float    oracle_fp16_to_f32(uint16_t h);
uint16_t oracle_f32_to_fp16(float f);
float    oracle_bf16_to_f32(uint16_t b);
uint16_t oracle_f32_to_bf16(float f);
void oracle_cast_f32_to_bf16(const float *src, uint16_t *dst, int n);
void oracle_cast_f32_to_fp16(const float *src, uint16_t *dst, int n);
void oracle_cast_bf16_to_f32(const uint16_t *src, float *dst, int n);
void oracle_cast_fp16_to_f32(const uint16_t *src, float *dst, int n);

/* ---- GEMMs: A[M,K] row-major times B[K,N] row-major ("NN") ---- */
/* n_threads <= 1 runs serially, otherwise a fork-join row split. */
void oracle_matmul_f32(const float *a, const float *b, float *c,
		       int M, int K, int N, int n_threads);
void oracle_matmul_bf16(const uint16_t *a, const uint16_t *b, uint16_t *c,
			int M, int K, int N, int n_threads);
void oracle_matmul_f16(const uint16_t *a, const uint16_t *b, uint16_t *c,
		       int M, int K, int N, int n_threads);
void oracle_matmul_f16_acc32(const uint16_t *a, const uint16_t *b,
			     uint16_t *c, int M, int K, int N, int n_threads);
void oracle_matmul_q8(const float *a, const void *b_blocks, float *c,
		      int M, int K, int N, int n_threads);

/* W stored [N,K] (PyTorch [out,in]) quantized flat, so blocks run along K. */
void oracle_matmul_q8_nt(const float *a, const void *w_blocks, float *c,
			 int M, int K, int N, int n_threads);

/* ---- 2-D transpose (src/backend/cpu/kernels/cpu_transpose.c:355-366) ---- */
void oracle_transpose_u16(const uint16_t *src, uint16_t *dst, int R, int C);
void oracle_transpose_f32(const float *src, float *dst, int R, int C);

/* ---- Epilogues (gh_linear / gh_mlp compose these after MATMUL) ---- */
void oracle_bias_add_f32(const float *x, const float *bias, float *out,
			 int rows, int N);
void oracle_bias_add_bf16(const uint16_t *x, const uint16_t *bias,
			  uint16_t *out, int rows, int N);
void oracle_bias_add_f16(const uint16_t *x, const uint16_t *bias,
			 uint16_t *out, int rows, int N);
void oracle_gelu_f32(const float *x, float *out, int n);
void oracle_gelu_bf16(const uint16_t *x, uint16_t *out, int n);
void oracle_gelu_f16(const uint16_t *x, uint16_t *out, int n);

/* ---- Batched (per-slice) bf16 matmul: loops the 2-D kernel ---- */
/* b_nt = 0: B slices are [K,N]; b_nt = 1: B slices are [N,K] and are
 * transposed per slice first, as gh_transpose + gh_matmul would. */
void oracle_matmul_bf16_batched(const uint16_t *a, const uint16_t *b,
				uint16_t *c, int batch, int M, int K, int N,
				int b_nt, int n_threads);

/* ---- SDPA (src/backend/cpu/kernels/cpu_sdpa.c:49-159, 216-288) ---- */
/* Q [BH,Sq,D], K/V [BH,Sk,D], mask [Sq,Sk] shared by all heads or NULL. */
void oracle_sdpa_f32(const float *q, const float *k, const float *v, const float *mask,
		     float *out, int BH, int Sq, int Sk, int D, int n_threads);

/* ---- LayerNorm over the last dim, eps 1e-5 (x86 scalar paths:
 * src/backend/cpu/kernels/cpu_layernorm.c:28-55, cpu_layernorm_bf16.c:
 * 88-115, cpu_layernorm_f16.c:99-127). gamma/beta of length cols or NULL,
 * in the input's dtype. ---- */
void oracle_layernorm_f32(const float *x, const float *gamma, const float *beta, float *out,
			  int rows, int cols, int n_threads);
void oracle_layernorm_bf16(const uint16_t *x, const uint16_t *gamma, const uint16_t *beta,
			   uint16_t *out, int rows, int cols, int n_threads);
void oracle_layernorm_f16(const uint16_t *x, const uint16_t *gamma, const uint16_t *beta,
			  uint16_t *out, int rows, int cols, int n_threads);

/* ---- RoPE, interleaved pairs (cpu_rope.c:88-104, cpu_rope_bf16.c:100-121,
 * cpu_rope_f16.c:100-121): x [batch, seq, heads, hd], cos/sin f32
 * [seq, hd/2]. ---- */
void oracle_rope_f32(const float *x, const float *cos_t, const float *sin_t, float *y,
		     int batch, int seq, int heads, int hd);
void oracle_rope_bf16(const uint16_t *x, const float *cos_t, const float *sin_t, uint16_t *y,
		      int batch, int seq, int heads, int hd);
void oracle_rope_f16(const uint16_t *x, const float *cos_t, const float *sin_t, uint16_t *y,
		     int batch, int seq, int heads, int hd);

/* ---- Conv2D NHWC x OHWI -> NHWC (cpu_conv2d.c:46-128, 296-435;
 * cpu_conv2d_bf16.c, cpu_conv2d_f16.c scalar paths): x [N,H,W,C], w
 * [OC,KH,KW,C/groups], y [N,OH,OW,OC]; f32 accumulation in im2col order,
 * 16-bit outputs rounded once. ---- */
void oracle_conv2d_f32(const float *x, const float *w, float *y, int N, int H, int W, int C,
		       int OC, int KH, int KW, int stride, int ph, int pw, int groups, int OH, int OW,
		       int n_threads);
void oracle_conv2d_bf16(const uint16_t *x, const uint16_t *w, uint16_t *y, int N, int H, int W,
			int C, int OC, int KH, int KW, int stride, int ph, int pw, int groups, int OH,
			int OW, int n_threads);
void oracle_conv2d_f16(const uint16_t *x, const uint16_t *w, uint16_t *y, int N, int H, int W,
		       int C, int OC, int KH, int KW, int stride, int ph, int pw, int groups, int OH,
		       int OW, int n_threads);

/* ---- ConvTranspose2D NHWC x OHWI (cpu_conv_transpose2d.c:55-131) and
 * MaxPool2D NHWC (cpu_maxpool2d.c:68-108), f32. ---- */
void oracle_conv_transpose2d_f32(const float *x, const float *w, float *y, int N, int H, int W,
				 int C, int OC, int KH, int KW, int stride, int pad, int n_threads);
void oracle_maxpool2d_f32(const float *x, float *y, int N, int H, int W, int C, int kernel,
			  int stride);

#endif /* SAM3_ORACLE_H */
