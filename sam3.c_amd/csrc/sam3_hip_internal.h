/*
 * sam3_hip_internal.h - helpers shared by the C11 host files of the HIP
 * backend (not part of the exported ABI).
 */
#ifndef SAM3_HIP_INTERNAL_H
#define SAM3_HIP_INTERNAL_H

#include "sam3_hip.h"

/* Record (and unless SAM3_HIP_QUIET, print) the last failure. */
void s3h_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

/* hipError_t -> sam3_error (OK / ENOMEM / EBACKEND), recording failures. */
enum sam3_error s3h_hip(int hip_error, const char *what);

size_t s3h_dtype_size(int dtype);
long long s3h_nelems(const struct sam3_tensor *t);
size_t s3h_tensor_bytes(const struct sam3_tensor *t);

/* SDPA node on device tensors with its output stored head-merged
 * ([B, Sq, H, D], the TRANSPOSE (0,2,1,3) of the node's output), as f32
 * or as the operand form fmt (S3H_A_PLANES / S3H_A_F16, f32 SDPA with
 * head size 64) of a GEMM reading rows of H*D. */
enum sam3_error s3h_sdpa_merged(const struct sam3_node *node, void *out, int fmt, unsigned *ovf,
				unsigned ovf_tag, void *stream);

/* Device-pointer elementwise nodes used by the dispatcher and graph_eval. */
enum sam3_error s3h_add(const struct sam3_node *node, void *stream);
enum sam3_error s3h_gelu(const struct sam3_node *node, void *stream);
enum sam3_error s3h_transpose(const struct sam3_node *node, void *stream);
int s3h_transpose_is_swap(const struct sam3_node *node);
/* f32 TRANSPOSE keeping its last axis, written as the operand form fmt
 * (S3H_A_PLANES / S3H_A_F16) of a GEMM reading the output as rows of K. */
int s3h_transpose_to_ok(const struct sam3_node *node, int K);
/* An f16 form (S3H_A_F16) stores ovf_tag to *ovf (when ovf is set) if
 * some values do not fit f16 (s3k_permute_to); the same holds for the
 * f16 output form of s3h_matmul_fmt_to. */
enum sam3_error s3h_transpose_to(const struct sam3_node *node, const void *src, void *dst, int fmt,
				 int K, unsigned *ovf, unsigned ovf_tag, void *stream);
/* Device scratch reused in stream order: a block given back with
 * s3h_scratch_free(p, stream) is handed out again only to requests on
 * that stream. s3h_scratch_release(stream) returns the stream's idle
 * blocks to the runtime (after synchronizing it). */
enum sam3_error s3h_scratch_alloc(void **p, size_t nbytes, void *stream);
enum sam3_error s3h_scratch_free(void *p, void *stream);
void s3h_scratch_release(void *stream);

/* ViT block ops on device pointers; the _ok forms say whether the node
 * runs on the GPU (dtypes and shapes), without reporting an error. */
int s3h_transpose_ok(const struct sam3_node *node);
int s3h_layernorm_ok(const struct sam3_node *node);
enum sam3_error s3h_layernorm(const struct sam3_node *node, void *stream);
int s3h_rope_ok(const struct sam3_node *node);
enum sam3_error s3h_rope(const struct sam3_node *node, void *stream);
int s3h_slice_ok(const struct sam3_node *node);
int s3h_cast_ok(const struct sam3_node *node);
enum sam3_error s3h_slice(const struct sam3_node *node, void *stream);
enum sam3_error s3h_reshape(const struct sam3_node *node);
/* Whether sam3_hip_kernel_sdpa takes this node (dtypes, ranks, head_dim). */
int s3h_sdpa_node_ok(const struct sam3_node *node);

/* CONV2D kernels (conv.hip) and BIAS_ADD. s3h_conv2d runs path 0 (the
 * best), S3H_CONV_IMPLICIT, _IM2COL or _DIRECT; bias/flags (S3K_EPI_*)
 * fold a following BIAS_ADD and GELU into the GEMM epilogue (paths 1-2). */
enum { S3H_CONV_IMPLICIT = 1, S3H_CONV_IM2COL = 2, S3H_CONV_DIRECT = 3 };
int s3h_conv2d_ok(const struct sam3_node *node);
int s3h_conv2d_path(const struct sam3_node *node);
enum sam3_error s3h_conv2d(const struct sam3_node *node, const void *bias, int flags, int path,
			   void *stream);
/* CONV_TRANSPOSE2D and MAXPOOL2D (NHWC, F32). s3h_conv_transpose2d runs
 * path 0 (the best), S3H_CONVT_GEMM (stride = KH = KW, pad 0: one GEMM and
 * a pixel-shuffle permute; bias/flags fold a BIAS_ADD and GELU) or
 * S3H_CONVT_DIRECT. */
enum { S3H_CONVT_GEMM = 1, S3H_CONVT_DIRECT = 3 };
int s3h_conv_transpose2d_ok(const struct sam3_node *node);
int s3h_conv_transpose2d_path(const struct sam3_node *node);
enum sam3_error s3h_conv_transpose2d(const struct sam3_node *node, const void *bias, int flags,
				     int path, void *stream);
int s3h_maxpool2d_ok(const struct sam3_node *node);
enum sam3_error s3h_maxpool2d(const struct sam3_node *node, void *stream);
int s3h_bias_add_ok(const struct sam3_node *node);
enum sam3_error s3h_bias_add(const struct sam3_node *node, void *stream);

/* The form matmul converts its A operand to before the GEMM, so the node
 * producing A can write that form directly: S3H_A_PLANES = bf16 [M, 3K]
 * [hi|lo|hi] (the split f32 GEMM), S3H_A_F16 = f16 [M, K] (the Q8 GEMM
 * with f32 activations). s3h_matmul_fmt runs the GEMM on A in that form. */
enum { S3H_A_PLAIN = 0, S3H_A_PLANES = 1, S3H_A_F16 = 2, S3H_A_LN = 3, S3H_A_ATT1 = 4 };
/* S3H_A_LN: A is the output of a LayerNorm that did not run; the skinny
 * Q8_0 GEMM normalizes its input rows itself (S3K_A_LN). With this form
 * the `a` argument of the s3h_matmul_* functions points to this host
 * struct of device pointers (gamma, beta may be NULL). */
struct s3h_ln_in {
	const float *x, *gamma, *beta;
};
/* Whether a Q8_0 GEMM (b on the device) can read A as the LayerNorm
 * input ln (f32 [M, K] rows): the streaming skinny kernel with
 * S3K_A_LN, the normalization bit-identical to the LayerNorm kernel's. */
int s3h_matmul_ln_ok(int b_dt, const void *b, int M, int N, int K, int flags,
		     const struct s3h_ln_in *ln);
/* S3H_A_ATT1: A is the head-merged output of an attention of one query
 * over one key per head (q, k, v [K / D heads, D] f32, mask: the entry
 * of that key, or NULL) that did not run; the f32 GEMV forms it from v
 * with the attention kernel's steps (S3K_A_ATT1). With this form the `a`
 * argument points to this host struct of device pointers. */
struct s3h_att1_in {
	const float *q, *k, *v, *mask;
	float scale;
	int D;
};
/* Whether a Q8_0 GEMM of one row (b on the device) can read A as at. */
int s3h_matmul_att1_ok(int b_dt, const void *b, int M, int N, int K, int flags,
		       const struct s3h_att1_in *at);
int s3h_matmul_a_format(int a_dt, const void *a, int b_dt, const void *b, int c_dt, int M, int N,
			int K, int flags);
enum sam3_error s3h_matmul_fmt(int a_fmt, int a_dt, const void *a, int b_dt, const void *b,
			       int c_dt, void *c, int M, int N, int K, const void *bias, int flags,
			       void *stream);
/* The same GEMM (f32 result) written directly as the operand form out_fmt
 * (S3H_A_PLANES / S3H_A_F16) of the GEMM that reads it next, or as f32
 * (S3H_A_PLAIN), with res (f32 [M, N], or NULL) added last, when
 * s3h_matmul_out_ok says its kernel can. row_map (f32 only; NULL or
 * {g, d1, d2}) stores C row m permuted as the s3k_gemm row map says. */
int s3h_matmul_out_ok(int a_fmt, int a_dt, const void *a, int b_dt, const void *b, int M, int N,
		      int K, int flags, int out_fmt);
/* Whether s3h_matmul_fmt_to can add an f32 [M, N] residual to the f32
 * result (S3H_A_PLAIN, no row map): the direct-to-LDS GEMM, or a skinny
 * Q8_0 GEMM. */
int s3h_matmul_res_ok(int a_fmt, int a_dt, const void *a, int b_dt, const void *b, int M, int N,
		      int K, int flags);
enum sam3_error s3h_matmul_fmt_to(int a_fmt, int out_fmt, int a_dt, const void *a, int b_dt,
				  const void *b, void *c, int M, int N, int K, const void *bias,
				  const void *res, const int *row_map, int flags, unsigned *ovf,
				  unsigned ovf_tag, unsigned *rowf, void *stream);
/* The attention operands of a fused qkv projection: the f32 result
 * [B*S, n_out*H*D] stored as n_out head-split tensors out[y] [B, H, S, D]
 * (columns y*H*D onward), RoPE (cos / sin [S, D/2]) applied to operand y
 * after the bias when bit y of rope is set (S3K_EPI_QKV). */
struct s3h_qkv {
	float *out[3];
	const float *cos_t, *sin_t;
	int S, H, D, rope;
};
/* Whether s3h_matmul_qkv can run this GEMM (s3h_matmul_fmt's, f32 out). */
int s3h_matmul_qkv_ok(int a_fmt, int a_dt, const void *a, int b_dt, const void *b, int M, int N,
		      int K, int flags, const struct s3h_qkv *q);
enum sam3_error s3h_matmul_qkv(int a_fmt, int a_dt, const void *a, int b_dt, const void *b, int M,
			       int N, int K, const void *bias, int flags, const struct s3h_qkv *q,
			       void *stream);

/* Prepared copies of constant weights (bf16 hi/lo planes, padded rows),
 * kept by the backend whose graph_eval is running on this thread. A copy
 * is keyed by the source's device address, the preparation (tag) and its
 * shape; it is kept only when the source lies in memory the backend knows
 * to be constant (a mapped weight range, or an uploaded input that no
 * node writes), and dropped with that memory. Outside graph_eval nothing
 * is cached. */
enum { S3H_PREP_SPLIT_W = 1,   /* f32 [rows, k] -> bf16 [rows, 3k] = [hi|hi|lo] */
       S3H_PREP_PAD_PLANES,    /* f32 [rows, K] -> bf16 [rows, 3k] over k >= K, zero padded */
       S3H_PREP_PAD16,         /* 16-bit [rows, K] -> [rows, k], zero padded */
       S3H_PREP_Q8_F16,        /* Q8_0 [rows, k] -> f16 [rows, k] (q*scale
				* over the row factor), then the factors f32 [rows] */
       S3H_PREP_CONVT_W,       /* OHWI [OC, taps, C] -> [taps*OC, C]           */
       S3H_PREP_Q8_CS };       /* Q8_0 [rows, k] -> weight-row factors f32 [rows] */
void *s3h_prep_find(const void *src, int tag, int rows, int k);
int s3h_prep_cacheable(const void *src, size_t src_bytes);
enum sam3_error s3h_prep_store(const void *src, int tag, int rows, int k, void *dev, size_t bytes);

/* Bulk host -> device copies through pinned staging buffers (upload.c).
 * Lanes and chunk size default to S3H_STAGE_LANES x S3H_STAGE_CHUNK_MB;
 * SAM3_HIP_UPLOAD_LANES / SAM3_HIP_UPLOAD_CHUNK_MB override them. */
#define S3H_STAGE_MAX_LANES 16
#define S3H_STAGE_LANES 8
#define S3H_STAGE_CHUNK_MB 4
struct s3h_stage_lane {
	void *stream;   /* hipStream_t */
	char *buf[2];   /* pinned, chunk bytes each */
	void *done[2];  /* hipEvent_t: the DMA out of buf[i] has finished */
};
struct s3h_stager {
	int device;
	int lanes;      /* 0 = not initialised */
	size_t chunk;
	struct s3h_stage_lane lane[S3H_STAGE_MAX_LANES];
};
enum sam3_error s3h_stager_init(struct s3h_stager *s, int device);
void s3h_stager_free(struct s3h_stager *s);
/* Copy nbytes from pageable host memory to dev; returns when the data is
 * in HBM. */
enum sam3_error s3h_stager_copy(struct s3h_stager *s, void *dev, const void *host, size_t nbytes);

#endif /* SAM3_HIP_INTERNAL_H */
