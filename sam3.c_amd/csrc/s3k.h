/*
 * s3k.h - launch interface between the C11 host (sam3_hip_backend.c) and
 * the HIP kernels (gemm.hip, skinny.hip, aux.hip).
 *
 * Everything here is plain C: the host side is compiled by gcc as C11,
 * the kernel side by hipcc for gfx950. Launchers return a hipError_t
 * value as int (0 = success) and never allocate device memory.
 */
#ifndef SAM3_S3K_H
#define SAM3_S3K_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element kinds; the numbering is sam3_dtype's (sam3_types.h:45-52). */
enum s3k_kind {
	S3K_F32  = 0,
	S3K_F16  = 1,
	S3K_BF16 = 2,
	S3K_Q8   = 5,
	/* output kinds only: f32 epilogue math, then the form the next GEMM
	 * reads: f16 [M, ldc], or bf16 planes [hi|lo|hi] with row pitch
	 * ldc = 3N (hi at n, lo at N + n, hi again at 2N + n) */
	S3K_C_F16OP  = 16,
	S3K_C_PLANES = 17,
};

/* Epilogue / layout flags. */
#define S3K_EPI_BIAS 1  /* out += bias[n] (bias has the output's kind)    */
#define S3K_EPI_GELU 2  /* out = tanh-GELU(out)                           */
#define S3K_B_NT     4  /* B stored [N,K] (k contiguous), else [K,N]      */
#define S3K_EPI_RES  8  /* out += res[m][n] last (res f32 [M,N]; kernels
			 * with the shared LDS epilogue only)             */
#define S3K_EPI_ROWSCALE 16 /* out = acc * rs[m] first: A holds row m of the
			     * activations times 1/rs[m] (a power of two,
			     * s3k_cast_f16_rows), so the f16 copy of rows
			     * outside the f16 range stays exact           */
#define S3K_EPI_QKV 32  /* f32 out, batch 1, direct-to-LDS GEMM only: the
			 * result is stored as the head-split attention
			 * operands (struct s3k_gemm, qkv_*) instead of C */
#define S3K_Q8_WAUTO 256 /* MFMA Q8 kernels (gemm_dlq8, gemm_dlpq) without
			  * S3K_EPI_COLSCALE: the kernel finds the weight-row
			  * factors itself (127 * the largest |scale| of each
			  * row, as s3k_q8_wfactors), running with factor 1 and
			  * again with the factors when a row of the tile needs
			  * one: the bits of the S3K_EPI_COLSCALE path */
#define S3K_A_LN    128 /* A holds a LayerNorm's f32 input rows: the kernel
			  * normalizes each row (eps 1e-5, gamma ln_g, beta
			  * ln_b, either NULL) with the LayerNorm kernel's
			  * arithmetic before use (q8_stream only) */
#define S3K_A_ATT1  512 /* A (one f32 row, batch 1) holds v of attention
			  * heads of one query and one key each (q, k, v
			  * [K / att_D heads, att_D]): the kernel forms the
			  * attention output from it, score = dot(q, k) *
			  * att_scale (+ att_mask[0]), p = expf(score - max),
			  * out = fmaf(p, v, 0) * (1 / p), with attn_generic's
			  * steps for a one-key row (q8_gemv only) */
#define S3K_EPI_COLSCALE 64 /* out = acc * cs[n] first (with the row factor):
			     * the weight-row factors of a Q8_0 weight
			     * (s3k_q8_wfactors). Kernels that round q*scale
			     * to f16 form f16(q * scale / cs[n]); on an f16
			     * copy of the weight made that way
			     * (s3k_q8_nk_to_f16_nk) only the epilogue
			     * multiply remains. The MFMA path requires it
			     * for Q8_0 weights; the skinny and generic
			     * kernels (q exact, scale in f32) reject it. */

/*
 * One (optionally strided-batched) GEMM: C[M,N] = A[M,K] * B, row-major.
 * A kind: F32 | F16 | BF16. B kind: F32 | F16 | BF16 | Q8 (Q8 must be
 * S3K_B_NT with K % 32 == 0: the rows of W[N,K] are whole 36-byte blocks).
 * C kind: F32 | F16 | BF16.  lda/ldb/ldc are in elements (for Q8 B the
 * row pitch is implied: K/32 blocks of 36 bytes).
 */
struct s3k_gemm {
	const void *a;
	const void *b;
	void       *c;
	const void *bias;
	int         M, N, K;
	int         lda, ldb, ldc;
	long long   stride_a, stride_b, stride_c; /* per batch: elements;
						   * bytes for a Q8 B      */
	int         batch;
	int         a_kind, b_kind, c_kind;
	int         flags;
	const void *res;                          /* S3K_EPI_RES: f32 [M, N] */
	/* row map (rm_g > 0): C row m is stored (and its residual read) at
	 * row ((a*rm_d2 + c)*rm_d1 + b)*rm_g + m % rm_g, where
	 * m / rm_g = (a*rm_d1 + b)*rm_d2 + c: the permute (0,2,1,3) of
	 * [., rm_d1, rm_d2, rm_g*N] applied to the output */
	int         rm_g, rm_d1, rm_d2;
	/* S3K_EPI_ROWSCALE: per-row f32 factors, rs[b * rs_sb + m] for
	 * batch slice b */
	const float *rs;
	long long   rs_sb;
	/* S3K_EPI_COLSCALE: per-column (weight-row) f32 factors, powers of
	 * two, cs[b * cs_sb + n] for batch slice b */
	const float *cs;
	long long   cs_sb;
	/* S3K_A_LN: LayerNorm gamma and beta, f32 [K], 16-byte aligned */
	const float *ln_g, *ln_b;
	/* S3K_A_ATT1: q and k f32 [K] (16-byte aligned), the mask entry of
	 * the query's one key (or NULL), the score scale, the head size */
	const float *att_q, *att_k, *att_mask;
	float        att_scale;
	int          att_D;
	/* f16 operand output (S3K_C_F16OP): when ovf is set, a value the f16
	 * copy cannot hold (|x| >= 2^15, finite) stores ovf_tag to *ovf; when
	 * rowf is set, output row m's parts store ovf_tag to rowf[2m] if they
	 * hold a value of |x| >= 2^-10 and to rowf[2m + 1] if their nonzero
	 * values all lie below it, so that s3k_rowflag_check finds the rows
	 * whose nonzero values are all below 2^-10 (their f16 copy would keep
	 * only a few bits) */
	unsigned   *ovf;
	unsigned    ovf_tag;
	unsigned   *rowf;
	/* S3K_EPI_QKV: with E = qkv_H * qkv_D, output column n of row m is
	 * element (b, s, h, d) = (m / qkv_S, m % qkv_S, (n % E) / qkv_D,
	 * n % qkv_D) of operand y = n / E and is stored at qkv_out[y] +
	 * ((b * qkv_H + h) * qkv_S + s) * qkv_D + d: the [B, H, S, D] head
	 * split. When bit y of qkv_rope is set, RoPE is applied to operand y
	 * after the bias: pairs (d, d + 1), cos / sin tables [qkv_S, qkv_D/2],
	 * products and sums rounded separately. qkv_D is a power of two
	 * >= 4, qkv_S >= 32, N = E, 2E or 3E, M a multiple of qkv_S. */
	float       *qkv_out[3];
	const float *qkv_cos, *qkv_sin;
	int          qkv_S, qkv_H, qkv_D, qkv_rope;
};

/* Which kernel s3k_gemm_launch would pick (for tests and the bench). */
enum s3k_path {
	S3K_PATH_NONE    = 0,
	S3K_PATH_MFMA    = 1, /* LDS-tiled MFMA GEMM                        */
	S3K_PATH_SKINNY  = 2, /* bandwidth-bound small-M Q8 kernel          */
	S3K_PATH_GENERIC = 3, /* one thread per output, reference order      */
};

int s3k_gemm_path(const struct s3k_gemm *g);
int s3k_gemm_launch(const struct s3k_gemm *g, void *stream);

/* Force one path (testing): returns hipErrorInvalidValue if it cannot run
 * this problem. */
int s3k_gemm_launch_path(const struct s3k_gemm *g, int path, void *stream);

/*
 * Weight-row factors of Q8_0 weights for kernels that round q*scale to
 * f16 (struct s3k_gemm, S3K_EPI_COLSCALE): for output column n, with
 * m the largest |q*scale| over the elements of weight row n (for a row
 * of whole blocks, 127 * its largest |block scale|: the same for blocks
 * of the quantizer, an upper bound otherwise), cs[n] = 2^e, e = 0 when m
 * lies in [2^-6, 2^15) or is 0, else the e that brings m into
 * [2^14, 2^15). The f16 values f16(q*scale*2^-e) then keep 11 bits, and
 * the f32 epilogue multiplies by 2^e, exactly. Batch slices of an [N,K]
 * weight (nt 1, blocks over the flat index n*K+k, any K) lie stride_b
 * bytes apart, cs[b*N + n]; nt 0 is one [K,N] weight with blocks over
 * k*N+n (the reference kernel contract), batch 1.
 */
int s3k_q8_wfactors(const void *blocks, float *cs, int K, int N, int nt, int batch,
		    long long stride_b, void *stream);
/*
 * Q8 [K,N] with blocks over the flat index k*N+n (the reference kernel
 * contract) -> f16 W^T[N,K], q*scale/cs[n] rounded to f16 (cs from
 * s3k_q8_wfactors with nt 0), so the Q8 NN case runs on the f16 NT GEMM
 * with S3K_EPI_COLSCALE. Any K, N.
 */
int s3k_q8_kn_to_f16_nk(const void *blocks, void *out, const float *cs, int K, int N,
			void *stream);
/* Q8 [N,K] with blocks over the flat index n*K+k (any K) -> f16 [N,K],
 * q*scale/cs[n] rounded to f16; the factors cs[N] are computed here and
 * stored (s3k_q8_wfactors' rule). */
int s3k_q8_nk_to_f16_nk(const void *blocks, void *out, float *cs, int K, int N,
			void *stream);

/* Elementwise ops the fused graph paths fall back to when they cannot
 * fuse (reference semantics, one rounding per op). */
/* Q8_0 quantize / dequantize of n f32 values (blocks over the flat index). */
int s3k_q8_quantize(const void *src, void *dst, int n, void *stream);
int s3k_q8_dequantize(const void *src, void *dst, int n, void *stream);
/* n values of kind src_kind -> dst_kind (F32, F16, BF16; kinds differ):
 * hw 0 by integer arithmetic, bit-exact with sam3.c's half.h; hw 1 by
 * the hardware conversions the GEMM epilogues use. */
int s3k_cast(int src_kind, int dst_kind, const void *src, void *dst, long long n, int hw,
	     void *stream);
/* n f32 or bf16 values -> f16 (RNE); 16-byte aligned pointers. */
int s3k_cast_f16(int kind, const void *src, void *dst, long long n, void *stream);
/* s3k_cast_f16_rows (one batch) and s3k_q8_nk_to_f16_nk of an [N, K]
 * weight (with its factors cs[N]) in one launch; hipErrorInvalidValue
 * when K % 32, K > 4096 or an alignment rules it out (then run the two
 * separately). */
int s3k_cast_rows_expand(int kind, const void *src, long long lda, void *dst, float *rs, int M,
			 int K, const void *wblk, void *wout, float *cs, int N, void *stream);
/*
 * Activations for a GEMM that rounds them to f16, row by row: batch
 * slices (at element stride sa) of M rows of K values (pitch lda) ->
 * dense f16 [batch, M, K] and row factors rs [batch, M]. A row whose
 * largest finite |x| lies in [2^-10, 2^15) (or is 0) is converted as is,
 * rs = 1; any other row is first multiplied by 2^-e, e chosen so that
 * its largest |x| lands in [2^14, 2^15), and rs = 2^e. The scaling is
 * exact, so a GEMM on the copy times rs equals the GEMM on the
 * activations up to the f16 rounding of in-range values.
 */
int s3k_cast_f16_rows(int kind, const void *src, long long lda, long long sa, void *dst,
		      float *rs, int batch, int M, int K, void *stream);
/* Fused attention out = softmax(Q K^T / sqrt(D) + mask) V over BH heads:
 * Q and out [BH, Sq, D], K and V [BH, Sk, D], one dtype (S3K_F32, _BF16,
 * _F16); mask f32 [Sq, Sk] or NULL. s3k_attn_path gives the kernel that
 * runs the problem (0 = none); s3k_attn runs it on `path` (0 = best:
 * S3K_ATTN_SMALL when it can run the problem with f32 output rows, else
 * that kernel). S3K_ATTN_SMALL: f32, D = 64, 1 <= Sk <= 128, 16-byte
 * aligned tensors, the latency-bound few-keys kernel. */
enum { S3K_ATTN_MFMA = 1, S3K_ATTN_GENERIC = 3, S3K_ATTN_SMALL = 4 };
int s3k_attn_path(int kind, const void *q, const void *k, const void *v, void *out,
		  int BH, int Sq, int Sk, int D);
int s3k_attn(int path, int kind, const void *q, const void *k, const void *v,
	     const float *mask, void *out, int BH, int Sq, int Sk, int D, void *stream);
/* s3k_attn with the heads merged in the output (oh > 0 heads per batch
 * item, oh | BH): head b*oh + h, query q is stored at row b*Sq + q,
 * columns h*D.., of [BH/oh * Sq, oh*D], the permute (0,2,1,3) of
 * [BH/oh, oh, Sq, D]. oh = 0 is s3k_attn. ofmt (f32 on the MFMA kernel
 * only): 0 f32 rows, S3K_LN_PLANES bf16 planes [hi|lo|hi] with row pitch
 * 3*oh*D, S3K_LN_F16 f16 rows storing ovf_tag to *ovf (when set) as
 * s3k_permute_to does: the merged rows as a GEMM's operand. */
int s3k_attn_heads(int path, int kind, const void *q, const void *k, const void *v,
		   const float *mask, void *out, int BH, int Sq, int Sk, int D, int oh,
		   int ofmt, unsigned *ovf, unsigned ovf_tag, void *stream);
/* The kernel s3k_attn_heads(0, ...) runs for these arguments (S3K_ATTN_*,
 * 0 when it refuses them). */
int s3k_attn_heads_path(int kind, const void *q, const void *k, const void *v, void *out, int BH,
			int Sq, int Sk, int D, int oh, int ofmt);
/* ViT block ops (blockops.hip). LayerNorm over the last dim of rows x
 * cols (gamma/beta of the input's kind or NULL, eps 1e-5); RoPE on
 * interleaved pairs of x [batch, seq, heads, hd] with f32 cos/sin
 * [seq, hd/2]; permutation of up to 4 axes (output axis k = input axis
 * axes[k]) of esize-byte elements. */
int s3k_layernorm(int kind, const void *x, const void *gamma, const void *beta, void *out,
		  long long rows, int cols, void *stream);
/* f32 LayerNorm written as the operand a GEMM reads: bf16 planes
 * [rows, 3*cols] = [hi|lo|hi] (S3K_LN_PLANES, the split f32 GEMM's A) or
 * f16 [rows, cols] (S3K_LN_F16, the Q8 GEMM's A); the same values as
 * s3k_layernorm followed by s3k_split3_bf16 / s3k_cast_f16. For the f16
 * form, ovf (when not NULL) receives ovf_tag if a row's largest |y| lies
 * outside [2^-10, 2^15) (and is not 0): the f16 copy of that row is not
 * faithful, and the caller redoes the GEMM on f32 values. */
enum { S3K_LN_SAME = 0, S3K_LN_PLANES = 1, S3K_LN_F16 = 2 };
int s3k_layernorm_to(int fmt, const float *x, const float *gamma, const float *beta, void *out,
		     long long rows, int cols, unsigned *ovf, unsigned ovf_tag, void *stream);
/* The same with output row m stored at the row map (rm_g, rm_d1, rm_d2)
 * of struct s3k_gemm (rm_g 0: identity): the ViT window partition. */
int s3k_layernorm_to_map(int fmt, const float *x, const float *gamma, const float *beta,
			 void *out, long long rows, int cols, int rm_g, int rm_d1, int rm_d2,
			 unsigned *ovf, unsigned ovf_tag, void *stream);
int s3k_rope(int kind, const void *x, const float *cos_t, const float *sin_t, void *out,
	     int batch, int seq, int heads, int hd, void *stream);
int s3k_permute(int esize, const void *src, void *dst, int ndim, const int *in_dims,
		const int *axes, void *stream);
/* f32 permute (last axis kept, its size % 4 == 0) written as the operand
 * of a GEMM that reads the output as rows of K values: fmt S3K_LN_PLANES
 * (bf16 [hi|lo|hi], row pitch 3K) or S3K_LN_F16 (ovf as for
 * s3k_layernorm_to, checked per 4 values: one past 2^15, or all nonzero
 * and below 2^-10). */
int s3k_permute_to(int fmt, const float *src, void *dst, int ndim, const int *in_dims,
		   const int *axes, int K, unsigned *ovf, unsigned ovf_tag, void *stream);
/* Stores tag to *ovf when some row of the n row-tag arrays flags[i]
 * (2 * rows[i] words each, as struct s3k_gemm's rowf) holds tag in its
 * second word and not in its first: a row whose nonzero values are all
 * below 2^-10. n <= 32 per call. */
int s3k_rowflag_check(int n, unsigned *const *flags, const int *rows, unsigned tag, unsigned *ovf,
		      void *stream);
/* Whether the skinny launch of g rounds its f32 / bf16 activations to f16
 * with per-row power-of-two factors inside the kernel (no row-scaled f16
 * copy needed first). */
int s3k_skinny_scales_rows(const struct s3k_gemm *g);
/* Whether the skinny kernels take g as it is (shape, kinds, alignment,
 * and for S3K_A_LN the streaming kernel's conditions). */
int s3k_skinny_ok(const struct s3k_gemm *g);
/* Whether a batched one-row skinny launch of g runs on the persistent
 * q8_gemv_tasks. */
int s3k_gemv_tasks_take(const struct s3k_gemm *g);
/* Whether a batched skinny launch of g (2-16 f16 activation rows) runs
 * on the persistent q8_stream_tasks. */
int s3k_stream_tasks_take(const struct s3k_gemm *g);
/* Attention operands [B, H, S, D] (f32), up to three (n_out) in one
 * launch: out[y] from columns col0[y].. of rows of `pitch` values holding
 * [B*S, H*D] (the q, k or v part of a fused qkv output), with RoPE
 * (tables [S, D/2]) where bit y of rope_mask is set. */
int s3k_rope_split3(const float *x, long long pitch, const long long *col0, const float *cos_t,
		    const float *sin_t, int rope_mask, float *const *out, int n_out, int B, int S,
		    int H, int D, void *stream);
/* f32 rows [rows, K] (pitch ld) -> bf16 [rows, 3K]: [hi, lo, hi] for
 * order 0, [hi, hi, lo] for order 1 (hi = bf16(x), lo = bf16(x - hi)). */
int s3k_split3_bf16(const float *src, void *dst, int rows, int K, long long ld, int order,
		    void *stream);
/* Whether the MFMA path of g (B Q8_0 [N,K]) runs the direct-to-LDS Q8
 * GEMM: f16 A directly, bf16 A after a cast to f16. */
int s3k_dlq8_eligible(const struct s3k_gemm *g);
/* Whether the direct-to-LDS bf16/f16 GEMM takes g (layout and alignment). */
int s3k_dl_eligible(const struct s3k_gemm *g);
int s3k_bias_add(int kind, const void *x, const void *bias, void *out,
		 long long rows, int n, void *stream);
int s3k_add_same(int kind, const void *x, const void *y, void *out,
		 long long n, void *stream);
int s3k_gelu(int kind, const void *x, void *out, long long n, void *stream);
/*
 * NHWC Conv2D (conv.hip): x [N,H,W,C], w OHWI [OC,KH,KW,C/groups],
 * y [N,OH,OW,OC], one kind for x, w, y (and bias, [OC], with
 * S3K_EPI_BIAS; S3K_EPI_GELU after it).
 *   s3k_conv_implicit: groups 1, C % 64 == 0; xa/wb are x and w for
 *     16-bit kinds, or their bf16 planes for f32 (x: [N*H*W, 3C] =
 *     [hi|lo|hi], w: [OC, 3K] = [hi|hi|lo], from s3k_split3_bf16);
 *     pixel_pitch = C or 3C.
 *   s3k_conv_im2col: the column matrix [M, Kp] (16-bit) or its f32 planes
 *     [M, 3Kp] for the GEMM, Kp >= KH*KW*C, Kp % 8 == 0 (zero padded);
 *     s3k_conv_wprep: the weight as [OC, Kp] or planes [OC, 3Kp].
 *   s3k_conv_direct: any groups; reference accumulation order.
 */
struct s3k_conv {
	const void *x;
	const void *w;
	void       *y;
	const void *bias;
	int kind, flags;
	int N, H, W, C, OC, KH, KW, stride, pad_h, pad_w, groups, OH, OW;
};
int s3k_conv_implicit(const struct s3k_conv *c, const void *xa, const void *wb, int pixel_pitch,
		      void *stream);
int s3k_conv_im2col(const struct s3k_conv *c, void *col, int Kp, void *stream);
int s3k_conv_wprep(int kind, const void *w, void *out, int OC, int K, int Kp, void *stream);
int s3k_conv_direct(const struct s3k_conv *c, void *stream);
/* ConvTranspose2D (reference gather order, bit-exact f32) and MaxPool2D,
 * NHWC f32 (neck.hip); b repeated `times` times. */
int s3k_conv_transpose_direct(const float *x, const float *w, float *y, int N, int H, int W, int C,
			      int OC, int KH, int KW, int stride, int pad, int OH, int OW,
			      void *stream);
int s3k_maxpool2d(const float *x, float *y, int N, int H, int W, int C, int kernel, int stride,
		  int OH, int OW, void *stream);
int s3k_repeat_f32(const float *b, float *out, int n, int times, void *stream);
/* batch slices of [rows, cols] -> [cols, rows] */
int s3k_transpose2d(int esize, const void *src, void *dst, int batch, int rows,
		    int cols, void *stream);

/*
 * The library's environment switches, parsed once (settings.c) and
 * re-read only by sam3_hip_reload_settings(). Tile overrides (-1 / 0 =
 * automatic choice) exist for measurements and tests; the fold switches
 * (1 = on) each turn one graph_eval fusion off when set to 0.
 */
struct s3h_settings {
	int dl_cfg, dlq8_cfg, conv_cfg;   /* SAM3_HIP_{DL,DLQ8,CONV}_CFG        */
	int attn_nw;                      /* SAM3_HIP_ATTN_NW: waves per SDPA wg */
	int attn_vdma;                    /* SAM3_HIP_ATTN_VDMA: 16-bit SDPA V tiles by
					   * direct-to-LDS loads (1, default) or
					   * through registers (0) */
	int sk_mr, sk_nt;                 /* SAM3_HIP_SK_CFG "mr,nt"             */
	int q8_expand;                    /* SAM3_HIP_Q8_EXPAND: -1 auto, 0, 1   */
	int q8_f32cast;                   /* SAM3_HIP_Q8_F32CAST                 */
	int q8_batch_path;                /* SAM3_HIP_Q8_BATCH_PATH: 0, 1, 2     */
	int f32_split;                    /* SAM3_HIP_F32_SPLIT                  */
	int unpartition_fold, residual_fold, gemm_operand, qkv_chain, ln_operand,
	    permute_operand, partition_fold, qkv_fold, sdpa_merge, ln_gemv_fold;
	int q8_wauto;                     /* SAM3_HIP_Q8_WAUTO: per-call weight-row
					   * factors found by the Q8 GEMM (1) or
					   * by a pass of their own (0)         */
	int att_gemv_fold;                /* SAM3_HIP_ATT_GEMV_FOLD: attention of
					   * one query over one key left to the
					   * Q8_0 GEMV reading its output      */
	int gemv_tasks;                   /* SAM3_HIP_GEMV_TASKS: batches of 1-16
					   * rows on the persistent q8_gemv_tasks
					   * and q8_stream_tasks (1) or one
					   * workgroup per task / the tiled GEMM */
	int gemv_f32;                     /* SAM3_HIP_GEMV_F32: one f32 activation
					   * row on the f32 VALU GEMV (1) or on
					   * the f16 MFMA stream (0)           */
	int readback_all;                 /* SAM3_HIP_READBACK=all               */
	int quiet;                        /* SAM3_HIP_QUIET set                  */
	int arena_mb;                     /* SAM3_HIP_ARENA_MB (0 = default)     */
};
const struct s3h_settings *s3h_settings(void);

/* The fixed device scratch of sam3_hip_matmul_q8_noalloc (noalloc.hip):
 * the current device's copy of a file-scope __device__ array, found with
 * hipGetSymbolAddress on a device's first call and kept per device.
 * *bytes is its size. Returns a hipError_t value. */
int s3k_noalloc_scratch(void **ptr, size_t *bytes);

#ifdef __cplusplus
}
#endif

#endif /* SAM3_S3K_H */
