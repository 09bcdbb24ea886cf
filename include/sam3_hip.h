/*
 * include/sam3_hip.h - MI355X (gfx950) matmul backend for sam3.c: C ABI.
 *
 * A drop-in for the matmul path of sam3.c's backend interface. Every
 * entry point is extern "C", takes plain pointers and sizes, and returns
 * enum sam3_error. Reference interfaces each one replaces are cited as
 * <path>:<line> in the sam3.c source tree.
 *
 * Pointers: the node-level kernels and the sam3_hip_matmul* entry points
 * take DEVICE pointers (HBM) and run asynchronously on `stream` (a
 * hipStream_t, NULL = the default stream); the stream plays the role the
 * CPU kernels' thread pool plays. The backend vtable (graph_eval) takes
 * sam3.c's ordinary graphs over host tensors and moves data itself.
 */
#ifndef SAM3_HIP_H
#define SAM3_HIP_H

#include "sam3_hip_abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ */
/* Backend object                                                       */
/* ------------------------------------------------------------------ */

/*
 * Ops table of the HIP backend. Replaces sam3_cpu_backend_ops()
 * (src/backend/cpu/cpu_backend.c:160-170) / sam3_metal_backend_ops()
 * (src/backend/metal/metal_backend.c:2114-2133) behind
 * struct sam3_backend_ops (src/backend/backend.h:31-56). graph_eval runs
 * MATMUL nodes (F32, F16, BF16, F32 x Q8_0) on the GPU, fusing
 * TRANSPOSE(W) -> MATMUL -> ADD(bias) -> GELU chains, and runs ADD,
 * GELU, TRANSPOSE, SDPA, LAYERNORM, ROPE, SLICE, CONV2D and
 * CONV_TRANSPOSE2D (with a following BIAS_ADD and GELU in their
 * epilogue), MAXPOOL2D and BIAS_ADD on the GPU as well
 * (RESHAPE is a view: no copy, no transfer); other ops go to the host
 * dispatcher set with sam3_hip_backend_set_host_dispatch, or fail with
 * SAM3_EDTYPE when none is set (as cpu_dispatch_node does for an op with
 * no kernel, src/backend/cpu/cpu_dispatch.c:664-669).
 */
const struct sam3_backend_ops *sam3_hip_backend_ops(void);

/*
 * Create and init a HIP backend on `device` (the role of
 * sam3_backend_init(SAM3_BACKEND_CPU), src/backend/backend.c:30-77).
 * Returns NULL on failure (no device, out of memory).
 */
struct sam3_backend *sam3_hip_backend_create(int device);

/* Free a backend made by sam3_hip_backend_create (backend.c:79-85). */
void sam3_hip_backend_destroy(struct sam3_backend *be);

/*
 * Host dispatcher for ops the HIP backend does not run: called with host
 * tensors, same signature role as cpu_dispatch_node
 * (src/backend/cpu/cpu_dispatch.c:591-686). In sam3.c this is a wrapper
 * around cpu_dispatch_node(node, scratch, pool).
 */
typedef enum sam3_error (*sam3_hip_host_dispatch_fn)(const struct sam3_node *node,
						     void *ctx);
void sam3_hip_backend_set_host_dispatch(struct sam3_backend *be,
					sam3_hip_host_dispatch_fn fn, void *ctx);

/* The backend's HIP stream (hipStream_t). */
void *sam3_hip_backend_stream(struct sam3_backend *be);

/* Counters of the last graph_eval (for tests and profiling). */
struct sam3_hip_eval_stats {
	int gpu_nodes;     /* nodes run by HIP kernels                        */
	int fused_nodes;   /* nodes folded into another node's kernel          */
	int host_nodes;    /* nodes handed to the host dispatcher              */
	int uploads;       /* host -> device copies                            */
	int cache_hits;    /* inputs found resident from an earlier eval       */
	int downloads;     /* device -> host copies                            */
	int mapped_reads;  /* inputs read from a range mapped by map_weights   */
	int prep_hits;     /* weights whose prepared copy (bf16 planes, padded
			    * rows) was reused instead of recomputed           */
	int operand_writes; /* LAYERNORM outputs written straight in the form
			     * their one consuming GEMM reads (not kept)      */
	int range_reruns;  /* 1 when a fused producer's f16 GEMM operand held
			    * values outside the f16 range and the graph was
			    * run again with f32 operands (then the counts
			    * above are the second run's)                   */
};
void sam3_hip_backend_last_stats(struct sam3_backend *be,
				 struct sam3_hip_eval_stats *out);

/* ------------------------------------------------------------------ */
/* Weights in HBM                                                       */
/* ------------------------------------------------------------------ */

/*
 * Copy a host range of weights into HBM once: in sam3.c, the data blob
 * of an open weight file, wf->data_base for wf->mapped_size minus the
 * blob's file offset (src/core/weight.c:303-474, format
 * docs/weight-format.md:68-98). Tensors made by sam3_weight_to_tensor
 * (weight.c:534-558) point into that blob, and graph_eval then reads each
 * input whose bytes lie inside a mapped range from the HBM copy at the
 * same offset, with no per-tensor upload (the per-tensor shadows that
 * replace the reference's direct reads of the mmap,
 * graph_helpers.c:122-145). The 64-byte tensor alignment of the file
 * carries over to HBM.
 *
 * The copy runs through pinned staging buffers on several host threads
 * and DMA queues; the call returns when the data is in HBM. The range
 * stays mapped until cache_invalidate touches any byte of it
 * (backend.h:50-55) or the backend is destroyed; arena_reset leaves it.
 * A range that overlaps a mapped one, or device memory, is SAM3_EINVAL.
 * No reference counterpart: the CPU backend reads the mmap directly.
 */
enum sam3_error sam3_hip_backend_map_weights(struct sam3_backend *be, const void *host,
					     size_t nbytes);

/* HBM address of host byte `host` inside a mapped range, else NULL. */
void *sam3_hip_backend_weight_ptr(struct sam3_backend *be, const void *host);

/*
 * Stack n_parts tensors of one dtype along dim 0 into a new tensor in HBM
 * ([d_i, cols] -> [sum d_i, cols], or 1-D [d_i] -> [sum d_i]): the QKV
 * weight and bias fusion of image_encoder.c:223-254 (fuse_3), also
 * decoder.c:93-140 and mask_decoder.c:47. fuse_3 declares its output F32
 * whatever the parts hold, so Q8_0 parts come out as F32-labelled block
 * bytes. Here the output keeps the parts' dtype: Q8_0 parts, each a whole
 * number of 32-element blocks, give the Q8_0 tensor of the stacked rows.
 *
 * Parts may be host memory, device memory or inside a mapped range (then
 * the copy stays in HBM). *out is filled: dtype, dims, strides (zero for
 * Q8_0, as weight.c:551-555), nbytes, and data = a device buffer the
 * backend owns until it is destroyed. Errors: NULL, rank other than 1-2,
 * column mismatch, or a Q8_0 part whose element count is not a multiple
 * of 32 -> SAM3_EINVAL; mixed dtypes -> SAM3_EDTYPE.
 */
enum sam3_error sam3_hip_backend_fuse_rows(struct sam3_backend *be,
					   const struct sam3_tensor *const *parts, int n_parts,
					   struct sam3_tensor *out);

/* ------------------------------------------------------------------ */
/* Node-level kernels. Same contract as the reference CPU kernels       */
/* (shapes from the last two dims, B = [K,N], K mismatch or output size */
/* mismatch -> SAM3_EINVAL, wrong dtypes -> SAM3_EINVAL), with device   */
/* data pointers and a stream in place of the thread pool.             */
/* ------------------------------------------------------------------ */

/* F32 [M,K] x F32 [K,N] -> F32. Replaces cpu_kernel_matmul
 * (src/backend/cpu/kernels/cpu_kernels.h:27-29, cpu_matmul.c:178-257). */
enum sam3_error sam3_hip_kernel_matmul(const struct sam3_node *node, void *stream);

/* F16 x F16 -> F16, f32 accumulation. Replaces cpu_kernel_matmul_f16
 * (cpu_kernels.h:90-91, cpu_matmul_f16.c:167-244), whose accumulator is
 * fp16; this kernel keeps f32 and rounds once. */
enum sam3_error sam3_hip_kernel_matmul_f16(const struct sam3_node *node, void *stream);

/* BF16 x BF16 -> BF16, f32 accumulation. Replaces cpu_kernel_matmul_bf16
 * (cpu_kernels.h:115-116, cpu_matmul_bf16.c:183-251). */
enum sam3_error sam3_hip_kernel_matmul_bf16(const struct sam3_node *node, void *stream);

/* F32 [M,K] x Q8_0 [K,N] (blocks over the flat index) -> F32. Replaces
 * cpu_kernel_matmul_q8 (cpu_kernels.h:134-135, cpu_matmul_q8.c:168-235). */
enum sam3_error sam3_hip_kernel_matmul_q8(const struct sam3_node *node, void *stream);

/* Fused attention, Q K V -> out = softmax(Q K^T / sqrt(hd) + mask) V.
 * Replaces cpu_kernel_sdpa (src/backend/cpu/kernels/cpu_kernels.h:221,
 * cpu_sdpa.c:216-288): same inputs (Q, K, V, optional mask [seq_q,
 * seq_k] shared by all heads), params[0] = head_dim, 2-D [seq, hd] or 4-D
 * [B, H, seq, hd] tensors. Q, K, V and out share one dtype (F32 as in the
 * reference, or F16/BF16); the mask is F32. Other ranks are SAM3_EINVAL
 * (the reference reads them as 2-D). */
enum sam3_error sam3_hip_kernel_sdpa(const struct sam3_node *node, void *stream);

/* The other ops of a ViT block (image_encoder.c:755-916 builds them
 * through graph_helpers.c:324-520,664-684), on device pointers:
 *   LAYERNORM over the last dim, eps 1e-5, optional gamma/beta of the
 *   input's dtype: replaces cpu_kernel_layernorm{,_f16,_bf16}
 *   (cpu_kernels.h, cpu_layernorm.c:198-254, cpu_layernorm_bf16.c,
 *   cpu_layernorm_f16.c); mean and variance are summed in another order,
 *   so f32 results agree to ~1e-6, not bit for bit.
 *   ROPE on interleaved pairs, x [batch, seq, heads, hd], cos/sin F32
 *   [seq, hd/2]: replaces cpu_kernel_rope{,_f16,_bf16} (cpu_rope.c:35-108);
 *   bit-identical.
 *   SLICE (params axis, start, end): replaces cpu_kernel_slice
 *   (cpu_slice.c:19-88).
 *   TRANSPOSE with params as the permutation of up to 4 axes (all zero:
 *   swap the last two): replaces cpu_kernel_transpose
 *   (cpu_transpose.c:313-387).
 *   RESHAPE: a view, output->data = input->data, as cpu_kernel_reshape
 *   (cpu_reshape.c:19-42). */
enum sam3_error sam3_hip_kernel_layernorm(const struct sam3_node *node, void *stream);
enum sam3_error sam3_hip_kernel_rope(const struct sam3_node *node, void *stream);
enum sam3_error sam3_hip_kernel_slice(const struct sam3_node *node, void *stream);
enum sam3_error sam3_hip_kernel_transpose(const struct sam3_node *node, void *stream);
enum sam3_error sam3_hip_kernel_reshape(const struct sam3_node *node);

/* CAST between F32, F16 and BF16: replaces cpu_kernel_cast
 * (src/backend/cpu/kernels/cpu_cast.c:162-215; the fp16/bf16 converters
 * of src/core/half.h:58-210). params[0] = target dtype, which must be the
 * output's (else SAM3_EINVAL); the same dtype is a copy; other pairs are
 * SAM3_EDTYPE. Bit-exact with half.h, NaN payloads included. */
enum sam3_error sam3_hip_kernel_cast(const struct sam3_node *node, void *stream);
/* The same on a forced conversion path: 1 = integer arithmetic (what
 * sam3_hip_kernel_cast runs), 2 = the hardware conversion instructions
 * the GEMM epilogues round with (v_cvt_pk_bf16_f32, v_cvt_f16_f32,
 * v_cvt_f32_f16). No reference counterpart: it exists to check those
 * instructions against half.h. */
enum sam3_error sam3_hip_cast_on_path(int path, const struct sam3_node *node, void *stream);

/*
 * CONV2D node kernel: cpu_kernel_conv2d (src/backend/cpu/kernels/
 * cpu_conv2d.c:296-435) and its twins cpu_kernel_conv2d_f16 / _bf16
 * (cpu_conv2d_f16.c, cpu_conv2d_bf16.c). Input [N,H,W,C] (NHWC), weight
 * OHWI [OC,KH,KW,C/groups], output [N,OH,OW,OC] with OH and OW read from
 * the output; params[0] = stride (<= 0 -> 1), [1] = pad_h, [2] = groups
 * (<= 0 -> 1), [3] = pad_w (0 -> pad_h). One dtype (F32, F16, BF16) for
 * input, weight and output, f32 accumulation, one rounding of the output.
 * Errors as the reference: NULL, non-4-D, channel or output-shape
 * mismatch -> SAM3_EINVAL; other dtypes or mixed ones -> SAM3_EDTYPE.
 *
 * Kernels: groups 1 with C % 64 == 0 runs an implicit GEMM on MFMA (the
 * column matrix is gathered in the load path, never written); other
 * groups-1 problems of >= 2^22 multiply-adds write the column matrix
 * and run the GEMM; the rest (groups, tiny problems) run one output per
 * thread in the reference's order (bit-exact for F32). F32 tensors run
 * the GEMMs as bf16 hi/lo splits (~1e-5 normwise; SAM3_HIP_F32_SPLIT=0
 * keeps them on the direct kernel).
 */
enum sam3_error sam3_hip_kernel_conv2d(const struct sam3_node *node, void *stream);

/* The kernel sam3_hip_kernel_conv2d picks (1 implicit GEMM, 2 column
 * matrix + GEMM, 3 direct; 0 if the node is invalid), and the conv on a
 * forced path (SAM3_EINVAL when that path cannot run it). No reference
 * counterpart: for tests and benches. */
int sam3_hip_conv2d_path(const struct sam3_node *node);
enum sam3_error sam3_hip_conv2d_on_path(int path, const struct sam3_node *node, void *stream);

/*
 * BIAS_ADD node kernel: cpu_kernel_bias_add / _bf16
 * (src/backend/cpu/kernels/cpu_bias_add.c:65-101, :150-190): x [.., C] +
 * bias [C] over the last dim, F32, BF16 (and F16), one dtype.
 */
enum sam3_error sam3_hip_kernel_bias_add(const struct sam3_node *node, void *stream);

/*
 * CONV_TRANSPOSE2D node kernel: cpu_kernel_conv_transpose2d
 * (src/backend/cpu/kernels/cpu_conv_transpose2d.c:140-217). Input
 * [N,H,W,C] (NHWC), weight OHWI [OC,KH,KW,C], output [N,OH,OW,OC] with
 * OH = (H-1)*stride - 2*pad + KH (and OW alike); params[0] = stride
 * (<= 0 -> 1), [1] = pad. F32 only, as the reference's dtype table
 * (cpu_dispatch.c:553-555): other dtypes -> SAM3_EDTYPE; channel or
 * output-shape mismatch -> SAM3_EINVAL. stride = KH = KW with no padding
 * (the neck's 2x2 upsampling) runs one GEMM over the input pixels and a
 * pixel-shuffle permute (bf16 hi/lo split GEMM, ~1e-5 normwise); other
 * shapes run the reference's gather order, bit-exact.
 */
enum sam3_error sam3_hip_kernel_conv_transpose2d(const struct sam3_node *node, void *stream);

/* The kernel sam3_hip_kernel_conv_transpose2d picks (1 GEMM, 3 direct; 0
 * if the node is invalid) and a forced one (SAM3_EINVAL if it cannot run
 * the node). No reference counterpart: for tests and benches. */
int sam3_hip_conv_transpose2d_path(const struct sam3_node *node);
enum sam3_error sam3_hip_conv_transpose2d_on_path(int path, const struct sam3_node *node,
						  void *stream);

/*
 * MAXPOOL2D node kernel: cpu_kernel_maxpool2d
 * (src/backend/cpu/kernels/cpu_maxpool2d.c:113-177). NHWC [N,H,W,C] ->
 * [N,OH,OW,C], params[0] = kernel (<= 0 -> 2), [1] = stride (<= 0 ->
 * kernel), OH = (H - kernel)/stride + 1; F32 only. The same scan as the
 * reference (first tap, then strictly greater ones), bit-exact, NaNs
 * included.
 */
enum sam3_error sam3_hip_kernel_maxpool2d(const struct sam3_node *node, void *stream);

/* Route one node by op and dtype. Replaces cpu_dispatch_node
 * (src/backend/cpu/cpu_dispatch.c:591-686): same mixed F32 x Q8_0 rule,
 * same SAM3_EDTYPE for mismatched dtypes or an (op, dtype) without a
 * kernel. Runs MATMUL, ADD, GELU, TRANSPOSE (up to 4 dims), SDPA,
 * LAYERNORM, ROPE (F32 cos/sin with any float input, as
 * cpu_dispatch.c:618-640), SLICE and RESHAPE. */
enum sam3_error sam3_hip_dispatch_node(const struct sam3_node *node, void *stream);

/* ------------------------------------------------------------------ */
/* Plain-pointer matmul. No counterpart in the reference: the node      */
/* kernels above unpack to these; they add the [N,K] weight layout, a   */
/* fused epilogue and strided batches, which the graph builder reaches  */
/* through TRANSPOSE/ADD/GELU nodes (src/model/graph_helpers.c:297-320, */
/* 1258-1276) and per-head attention slices (graph_helpers.c:808-843).  */
/* ------------------------------------------------------------------ */
#define SAM3_HIP_BIAS 1   /* C += bias[N] (bias dtype = c_dtype)           */
#define SAM3_HIP_GELU 2   /* C = tanh-GELU(C) (cpu_gelu.c:23-38)            */
#define SAM3_HIP_B_NT 4   /* B stored [N,K] (PyTorch [out,in]); else [K,N]  */

/*
 * C[M,N] = A[M,K] * B (+bias) (GELU). Dtypes are enum sam3_dtype:
 *   a F32/F16/BF16 with b of the same dtype, c = a's dtype or F32;
 *   a F32/F16/BF16 with b Q8_0, c F32. Q8_0 B is [K,N] with
 *   blocks over the flat index (the kernel contract) or, with
 *   SAM3_HIP_B_NT, W[N,K] quantized flat (blocks along K).
 * Rows are dense (lda = K, ldb = N or K, ldc = N).
 */
enum sam3_error sam3_hip_matmul(int a_dtype, const void *a,
				int b_dtype, const void *b,
				int c_dtype, void *c,
				int M, int N, int K,
				const void *bias, int flags, void *stream);

/*
 * Strided batch: for s in [0, batch): C_s = A_s * B_s, with element
 * strides stride_a/b/c between slices (bytes for a Q8_0 B). dtype is F16
 * or BF16 (c has the same dtype) or F32. With SAM3_HIP_B_NT, B_s is
 * [N,K] (attention's Q K^T), else [K,N] (attention's P V).
 */
enum sam3_error sam3_hip_matmul_batched(int dtype, const void *a, const void *b, void *c,
					int batch, int M, int N, int K,
					long long stride_a, long long stride_b,
					long long stride_c, int flags, void *stream);

/*
 * Strided batch of Q8_0 weight matmuls: for s in [0, batch),
 * C_s[M,N] (F32) = A_s[M,K] * W_s^T (+bias) (GELU), with W_s[N,K] Q8_0
 * blocks along k (K % 32 == 0) at a byte stride stride_w, A_s at element
 * stride stride_a (a_dtype F32, F16 or BF16), C_s at element stride
 * stride_c, one bias[N] (F32) for every slice. Small M (<= 128) runs as
 * one launch of the bandwidth-bound kernel over all slices; otherwise one
 * launch per slice. No counterpart in the reference: it runs a stream of
 * layers' or heads' weights (graph_helpers.c:297-320 once per weight)
 * without a launch per weight. flags: SAM3_HIP_BIAS | SAM3_HIP_GELU.
 */
enum sam3_error sam3_hip_matmul_q8_batched(int a_dtype, const void *a, const void *w,
					   void *c, int batch, int M, int N, int K,
					   long long stride_a, long long stride_w,
					   long long stride_c, const void *bias, int flags,
					   void *stream);

/*
 * sam3_hip_matmul for Q8_0 weights that allocates nothing: C[M,N] (F32) =
 * A[M,K] * W^T (+bias) (GELU), W[N,K] Q8_0 blocks along k (K % 32 == 0),
 * A F32, F16 or BF16, bias F32 [N]. It runs the kernels of
 * sam3_hip_matmul with per-call weight expansion off (SAM3_HIP_Q8_EXPAND=0):
 * the same bits as that setting; at the default setting sam3_hip_matmul
 * expands large weights to f16 first, and the two agree within the f32
 * tolerance. The f16 copy of f32/bf16 activations and the weight-row
 * factors of the MFMA kernels go to a fixed scratch array of 48 MiB that
 * the library keeps on each device until the process ends; a problem
 * needing more (M * K * 2 bytes plus 4 per row, rounded up to 256, plus
 * 4 * N) fails with SAM3_EINVAL before any launch. No hipMalloc,
 * hipFree or other allocation happens. Calls that overlap on one device
 * (from two threads or on two streams) share the array and race.
 * No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops).
 * flags: SAM3_HIP_BIAS | SAM3_HIP_GELU (W is always [N,K]).
 */
enum sam3_error sam3_hip_matmul_q8_noalloc(int a_dtype, const void *a, const void *w, void *c,
					   int M, int N, int K, const void *bias, int flags,
					   void *stream);

/* Which kernel sam3_hip_matmul would launch for this problem:
 * 1 = tiled MFMA, 2 = skinny (small-M Q8), 3 = generic, 0 = none. */
int sam3_hip_matmul_path(int a_dtype, int b_dtype, int c_dtype,
			 int M, int N, int K, int flags);

/* sam3_hip_matmul on a forced kernel path (1, 2 or 3 as above), for
 * cross-checking the paths against each other. SAM3_EINVAL if that path
 * cannot run the problem. */
enum sam3_error sam3_hip_matmul_on_path(int path, int a_dtype, const void *a,
					int b_dtype, const void *b,
					int c_dtype, void *c,
					int M, int N, int K,
					const void *bias, int flags, void *stream);

/* ------------------------------------------------------------------ */
/* Plain-pointer attention (device pointers, async on `stream`).        */
/* ------------------------------------------------------------------ */

/* out[h] = softmax(q[h] k[h]^T / sqrt(D) + mask) v[h] for h < BH, the
 * computation of cpu_kernel_sdpa (cpu_sdpa.c:49-159 per query row):
 * q and out [BH, Sq, D], k and v [BH, Sk, D], contiguous, all of `dtype`
 * (SAM3_DTYPE_F32, _F16 or _BF16); mask f32 [Sq, Sk] or NULL. A query
 * whose scores are all -inf gets zeros, as there. D = 64 with 16-byte
 * aligned tensors runs the MFMA kernel (f32 as three bf16 products per
 * step: hi*hi + lo*hi + hi*lo), or for f32 with at most 128 keys a
 * latency-bound kernel in plain f32 arithmetic (the text encoder's
 * attention); other D up to 512 run a one-wave-per-row f32 kernel. */
enum sam3_error sam3_hip_sdpa(int dtype, const void *q, const void *k, const void *v,
			      const float *mask, void *out, int BH, int Sq, int Sk, int D,
			      void *stream);

/* sam3_hip_sdpa on a forced kernel: 0 = best, 1 = MFMA (D = 64), 3 = the
 * any-D kernel, 4 = the few-keys kernel (f32, D = 64, Sk <= 128, 16-byte
 * aligned). SAM3_EINVAL if that kernel cannot run the problem. */
enum sam3_error sam3_hip_sdpa_on_path(int path, int dtype, const void *q, const void *k,
				      const void *v, const float *mask, void *out, int BH,
				      int Sq, int Sk, int D, void *stream);

/* ------------------------------------------------------------------ */
/* Q8_0 format on the device (device pointers, async on `stream`).      */
/* ------------------------------------------------------------------ */

/* Quantize nelems f32 values into ceil(nelems/32) 36-byte blocks over the
 * flat index. Replaces sam3_q8_quantize (src/core/quant.c:67-130),
 * bit-exact with its x86 build (roundf, halves away from zero). Pointers
 * 4-byte aligned. */
enum sam3_error sam3_hip_q8_quantize(const float *src, void *dst_blocks, int nelems,
				     void *stream);

/* x = (float)q * scale for nelems values. Replaces sam3_q8_dequantize
 * (src/core/quant.c:134-165). Pointers 4-byte aligned. */
enum sam3_error sam3_hip_q8_dequantize(const void *src_blocks, float *dst, int nelems,
				       void *stream);

/* ------------------------------------------------------------------ */
/* Device memory, streams and events for FFI callers (no counterpart    */
/* in the reference, whose tensors are host memory).                    */
/* ------------------------------------------------------------------ */
int  sam3_hip_device_count(void);
enum sam3_error sam3_hip_set_device(int device);
enum sam3_error sam3_hip_malloc(void **ptr, size_t nbytes);
enum sam3_error sam3_hip_free(void *ptr);
enum sam3_error sam3_hip_memcpy_h2d(void *dst, const void *src, size_t nbytes);
enum sam3_error sam3_hip_memcpy_d2h(void *dst, const void *src, size_t nbytes);
enum sam3_error sam3_hip_memcpy_d2d(void *dst, const void *src, size_t nbytes);
enum sam3_error sam3_hip_synchronize(void);
enum sam3_error sam3_hip_stream_create(void **stream);
/* Also frees the device scratch the library keeps for this stream (after
 * the stream's work completes). */
enum sam3_error sam3_hip_stream_destroy(void *stream);
enum sam3_error sam3_hip_stream_synchronize(void *stream);
enum sam3_error sam3_hip_event_create(void **event);
enum sam3_error sam3_hip_event_destroy(void *event);
enum sam3_error sam3_hip_event_record(void *event, void *stream);
enum sam3_error sam3_hip_event_elapsed_ms(float *ms, void *start, void *stop);
/* gcnArchName of the device (e.g. "gfx950:sramecc+:xnack-"), or "". */
const char *sam3_hip_device_arch(int device);
/* Message of the last failure on this thread ("" if none). */
const char *sam3_hip_last_error(void);
/* Re-read the SAM3_HIP_* environment switches (tile overrides, graph_eval
 * fold switches). They are parsed once, at first use; call this after
 * changing the environment, while no other thread launches work. No
 * reference counterpart (the reference has no such switches). */
enum sam3_error sam3_hip_reload_settings(void);

#ifdef __cplusplus
}
#endif

#endif /* SAM3_HIP_H */
