/*
 * oracle/sam3_oracle.c - CPU restatement of sam3.c's matmul path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and CPU baseline ("port")
 * for the HIP backend. Nothing in the product path calls this file.
 *
 * Each routine restates the x86 scalar branch of the cited reference
 * code with the same per-element operation order (no FP contraction,
 * built -std=c11 -O2 -ffp-contract=off), so outputs are bit-identical to
 * the reference's own x86 build. Paths are relative to /root/reference.
 *
 * Parity pins, per function (tests/test_oracle.py):
 *   q8 quantize/dequantize, block count/nbytes: golden vectors from the
 *     reference, direct _ref comparison, tests/test_quant.c known answers,
 *     |q| <= 127 and scale == amax/127 invariants.
 *   fp16/bf16 conversions: exhaustive 65536-pattern sweeps and a 2^20
 *     f32 sweep against _ref's cpu_kernel_cast; golden vectors.
 *   matmul f32/bf16/f16/q8: golden vectors, _ref comparison, the
 *     reference tests' known answers (58,64,139,154; identity), one-hot
 *     rows and float64 brute force.
 *   matmul_q8_nt: per output column it must equal the reference Q8
 *     kernel run with B = W[n,:] viewed as [K,1] (same memory, same
 *     arithmetic); checked bit-exactly against _ref and golden vectors.
 *   matmul_f16_acc32 (no reference counterpart: the reference f16 GEMM
 *     accumulates in fp16): pinned by float64 brute force, by equality
 *     with the bf16 kernel's structure on inputs exactly representable in
 *     both formats, and by identity/one-hot closed forms.
 *   bias add / gelu: golden vectors and _ref comparison.
 *   batched bf16: per-slice equality with the 2-D kernel and _ref.
 */
#include "sam3_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* Bit casts (src/core/half.h:33-47 use memcpy for the same purpose).   */
/* ------------------------------------------------------------------ */
static inline float bits_to_f32(uint32_t u)
{
	float f;
	memcpy(&f, &u, 4);
	return f;
}

static inline uint32_t f32_to_bits(float f)
{
	uint32_t u;
	memcpy(&u, &f, 4);
	return u;
}

/* ------------------------------------------------------------------ */
/* fp16 <-> f32 (src/core/half.h:58-161)                               */
/* ------------------------------------------------------------------ */
float oracle_fp16_to_f32(uint16_t h)
{
	uint32_t s = (uint32_t)(h & 0x8000u) << 16;
	uint32_t e = (h >> 10) & 0x1Fu;
	uint32_t m = h & 0x3FFu;

	if (e == 0x1Fu)                       /* inf / nan */
		return bits_to_f32(s | 0x7F800000u | (m << 13));
	if (e != 0u)                          /* normal: rebias 15 -> 127 */
		return bits_to_f32(s | ((e + 112u) << 23) | (m << 13));
	if (m == 0u)                          /* signed zero */
		return bits_to_f32(s);
	/* subnormal: shift the leading one up to bit 10 */
	uint32_t e32 = 113u;
	while (!(m & 0x400u)) {
		m <<= 1;
		e32--;
	}
	return bits_to_f32(s | (e32 << 23) | ((m & 0x3FFu) << 13));
}

uint16_t oracle_f32_to_fp16(float f)
{
	uint32_t u = f32_to_bits(f);
	uint32_t s = (u >> 16) & 0x8000u;
	uint32_t e8 = (u >> 23) & 0xFFu;
	uint32_t m = u & 0x7FFFFFu;
	int32_t e = (int32_t)e8 - 112;        /* rebias 127 -> 15 */

	if (e >= 31) {
		if (e8 == 0xFFu)              /* inf, or nan with payload kept */
			return (uint16_t)(s | 0x7C00u |
					  (m ? ((m >> 13) | 1u) : 0u));
		return (uint16_t)(s | 0x7C00u);  /* overflow */
	}
	if (e <= 0) {
		if (e < -10)
			return (uint16_t)s;   /* underflow to signed zero */
		m = (m | 0x800000u) >> (1 - e);
		uint32_t half = m & 0x1000u, rest = m & 0x0FFFu;
		m >>= 13;
		if (half && (rest || (m & 1u)))
			m++;          /* may carry into the smallest normal */
		return (uint16_t)(s | m);
	}
	uint32_t half = m & 0x1000u, rest = m & 0x0FFFu;
	m >>= 13;
	if (half && (rest || (m & 1u))) {
		m++;
		if (m == 0x400u) {
			m = 0;
			if (++e >= 31)
				return (uint16_t)(s | 0x7C00u);
		}
	}
	return (uint16_t)(s | ((uint32_t)e << 10) | m);
}

/* ------------------------------------------------------------------ */
/* bf16 <-> f32 (src/core/half.h:173-210)                              */
/* ------------------------------------------------------------------ */
float oracle_bf16_to_f32(uint16_t b)
{
	return bits_to_f32((uint32_t)b << 16);
}

uint16_t oracle_f32_to_bf16(float f)
{
	uint32_t u = f32_to_bits(f);

	if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu))
		return (uint16_t)((u >> 16) | 0x40u);   /* quiet NaN */
	uint32_t t = u >> 16;
	if (((u >> 15) & 1u) && ((u & 0x7FFFu) || (t & 1u)))
		t++;                                    /* round half even */
	return (uint16_t)t;
}

void oracle_cast_f32_to_bf16(const float *src, uint16_t *dst, int n)
{
	for (int i = 0; i < n; i++)
		dst[i] = oracle_f32_to_bf16(src[i]);
}

void oracle_cast_f32_to_fp16(const float *src, uint16_t *dst, int n)
{
	for (int i = 0; i < n; i++)
		dst[i] = oracle_f32_to_fp16(src[i]);
}

void oracle_cast_bf16_to_f32(const uint16_t *src, float *dst, int n)
{
	for (int i = 0; i < n; i++)
		dst[i] = oracle_bf16_to_f32(src[i]);
}

void oracle_cast_fp16_to_f32(const uint16_t *src, float *dst, int n)
{
	for (int i = 0; i < n; i++)
		dst[i] = oracle_fp16_to_f32(src[i]);
}

/* ------------------------------------------------------------------ */
/* Q8_0 (src/core/quant.h:22-33, src/core/quant.c:29-165)              */
/* A block is 36 bytes: f32 scale then 32 int8 values.                  */
/* ------------------------------------------------------------------ */
struct q8blk {
	float  d;
	int8_t q[ORACLE_Q8_BLOCK];
};

int oracle_q8_block_count(int nelems)
{
	return (nelems + ORACLE_Q8_BLOCK - 1) / ORACLE_Q8_BLOCK;
}

size_t oracle_q8_nbytes(int nelems)
{
	return (size_t)oracle_q8_block_count(nelems) * sizeof(struct q8blk);
}

/* x86 branch of quant.c:67-130: amax by fabsf, scale = amax/127,
 * q = clamp((int)roundf(x * (1/scale)), -127, 127); zero block -> all 0. */
void oracle_q8_quantize(const float *src, void *dst_blocks, int nelems)
{
	struct q8blk *dst = dst_blocks;
	int nb = oracle_q8_block_count(nelems);

	for (int b = 0; b < nb; b++) {
		const float *x = src + (size_t)b * ORACLE_Q8_BLOCK;
		int n = nelems - b * ORACLE_Q8_BLOCK;
		if (n > ORACLE_Q8_BLOCK)
			n = ORACLE_Q8_BLOCK;

		float amax = 0.0f;
		for (int i = 0; i < n; i++)
			if (fabsf(x[i]) > amax)
				amax = fabsf(x[i]);

		struct q8blk *o = &dst[b];
		o->d = amax / 127.0f;
		memset(o->q, 0, sizeof(o->q));
		if (o->d == 0.0f)
			continue;

		float inv = 1.0f / o->d;
		for (int i = 0; i < n; i++) {
			int v = (int)roundf(x[i] * inv);
			o->q[i] = (int8_t)(v > 127 ? 127 : (v < -127 ? -127 : v));
		}
	}
}

/* quant.c:134-165: x = (float)q * scale. */
void oracle_q8_dequantize(const void *src_blocks, float *dst, int nelems)
{
	const struct q8blk *src = src_blocks;

	for (int i = 0; i < nelems; i++) {
		const struct q8blk *blk = &src[i / ORACLE_Q8_BLOCK];
		dst[i] = (float)blk->q[i % ORACLE_Q8_BLOCK] * blk->d;
	}
}

/* ------------------------------------------------------------------ */
/* Fork-join row split, as sam3_threadpool_parallel_for drives the      */
/* kernels (src/util/threadpool.c:236-281 with the per-kernel split     */
/* chunk = M / n_tasks, last task takes the remainder, e.g.             */
/* src/backend/cpu/kernels/cpu_matmul_q8.c:145-157). Rows are           */
/* independent, so the split never changes results.                     */
/* ------------------------------------------------------------------ */
typedef void (*rows_fn)(void *ctx, int m0, int m1);

struct split_task {
	rows_fn fn;
	void   *ctx;
	int     m0, m1;
};

static void *split_worker(void *arg)
{
	struct split_task *t = arg;
	t->fn(t->ctx, t->m0, t->m1);
	return NULL;
}

static void run_rows(rows_fn fn, void *ctx, int M, int n_threads)
{
	if (n_threads <= 1 || M < 2) {
		fn(ctx, 0, M);
		return;
	}
	if (n_threads > 256)
		n_threads = 256;

	struct split_task tasks[256];
	pthread_t tids[256];
	int chunk = M / n_threads;

	for (int t = 0; t < n_threads; t++) {
		tasks[t].fn = fn;
		tasks[t].ctx = ctx;
		tasks[t].m0 = t * chunk;
		tasks[t].m1 = (t == n_threads - 1) ? M : (t + 1) * chunk;
	}
	int started[256] = {0};
	for (int t = 1; t < n_threads; t++)
		if (tasks[t].m0 < tasks[t].m1)
			started[t] = pthread_create(&tids[t], NULL,
						    split_worker, &tasks[t]) == 0;
	/* the caller runs task 0, and any task whose thread failed */
	if (tasks[0].m0 < tasks[0].m1)
		fn(ctx, tasks[0].m0, tasks[0].m1);
	for (int t = 1; t < n_threads; t++) {
		if (started[t])
			pthread_join(tids[t], NULL);
		else if (tasks[t].m0 < tasks[t].m1)
			fn(ctx, tasks[t].m0, tasks[t].m1);
	}
}

struct mm_ctx {
	const void *a, *b;
	void       *c;
	int         M, K, N;
};

/* Tile sizes of the reference kernels (cpu_matmul*.c: TILE_M/N/K). */
#define TM 8
#define TN 8
#define TK 64

static inline int imin(int x, int y) { return x < y ? x : y; }

/* ---- f32: cpu_matmul.c:40-63 (scalar; C zeroed, then c += a*b) ---- */
static void mm_f32_rows(void *p, int m0, int m1)
{
	struct mm_ctx *x = p;
	const float *a = x->a, *b = x->b;
	float *c = x->c;
	int K = x->K, N = x->N;

	memset(c + (size_t)m0 * N, 0, (size_t)(m1 - m0) * N * sizeof(float));
	for (int i0 = m0; i0 < m1; i0 += TM)
		for (int j0 = 0; j0 < N; j0 += TN)
			for (int k0 = 0; k0 < K; k0 += TK)
				for (int i = i0; i < imin(i0 + TM, m1); i++)
					for (int k = k0; k < imin(k0 + TK, K); k++) {
						float av = a[(size_t)i * K + k];
						for (int j = j0; j < imin(j0 + TN, N); j++)
							c[(size_t)i * N + j] +=
								av * b[(size_t)k * N + j];
					}
}

void oracle_matmul_f32(const float *a, const float *b, float *c,
		       int M, int K, int N, int n_threads)
{
	struct mm_ctx x = { a, b, c, M, K, N };
	run_rows(mm_f32_rows, &x, M, n_threads);
}

/* ---- bf16: cpu_matmul_bf16.c:103-141 (f32 tile acc, one RNE out) ---- */
static void mm_bf16_rows(void *p, int m0, int m1)
{
	struct mm_ctx *x = p;
	const uint16_t *a = x->a, *b = x->b;
	uint16_t *c = x->c;
	int K = x->K, N = x->N;

	for (int i0 = m0; i0 < m1; i0 += TM) {
		int i1 = imin(i0 + TM, m1);
		for (int j0 = 0; j0 < N; j0 += TN) {
			int j1 = imin(j0 + TN, N);
			float acc[TM][TN] = {{0}};
			for (int k0 = 0; k0 < K; k0 += TK)
				for (int i = i0; i < i1; i++)
					for (int k = k0; k < imin(k0 + TK, K); k++) {
						float av = oracle_bf16_to_f32(
							a[(size_t)i * K + k]);
						for (int j = j0; j < j1; j++)
							acc[i - i0][j - j0] += av *
								oracle_bf16_to_f32(
								b[(size_t)k * N + j]);
					}
			for (int i = i0; i < i1; i++)
				for (int j = j0; j < j1; j++)
					c[(size_t)i * N + j] =
						oracle_f32_to_bf16(acc[i - i0][j - j0]);
		}
	}
}

void oracle_matmul_bf16(const uint16_t *a, const uint16_t *b, uint16_t *c,
			int M, int K, int N, int n_threads)
{
	struct mm_ctx x = { a, b, c, M, K, N };
	run_rows(mm_bf16_rows, &x, M, n_threads);
}

/* ---- f16: cpu_matmul_f16.c:73-101 (fp16 accumulator, rounded each k) ---- */
static void mm_f16_rows(void *p, int m0, int m1)
{
	struct mm_ctx *x = p;
	const uint16_t *a = x->a, *b = x->b;
	uint16_t *c = x->c;
	int K = x->K, N = x->N;

	memset(c + (size_t)m0 * N, 0, (size_t)(m1 - m0) * N * sizeof(uint16_t));
	for (int i0 = m0; i0 < m1; i0 += TM)
		for (int j0 = 0; j0 < N; j0 += TN)
			for (int k0 = 0; k0 < K; k0 += TK)
				for (int i = i0; i < imin(i0 + TM, m1); i++)
					for (int k = k0; k < imin(k0 + TK, K); k++) {
						float av = oracle_fp16_to_f32(
							a[(size_t)i * K + k]);
						for (int j = j0; j < imin(j0 + TN, N); j++) {
							uint16_t *cp = &c[(size_t)i * N + j];
							float cur = oracle_fp16_to_f32(*cp);
							float bv = oracle_fp16_to_f32(
								b[(size_t)k * N + j]);
							*cp = oracle_f32_to_fp16(cur + av * bv);
						}
					}
}

void oracle_matmul_f16(const uint16_t *a, const uint16_t *b, uint16_t *c,
		       int M, int K, int N, int n_threads)
{
	struct mm_ctx x = { a, b, c, M, K, N };
	run_rows(mm_f16_rows, &x, M, n_threads);
}

/* ---- f16 with an f32 accumulator: the bf16 kernel's structure
 * (cpu_matmul_bf16.c:103-141) with the fp16 converters of half.h. No
 * reference kernel computes this; it is the f16 parity target. ---- */
static void mm_f16acc32_rows(void *p, int m0, int m1)
{
	struct mm_ctx *x = p;
	const uint16_t *a = x->a, *b = x->b;
	uint16_t *c = x->c;
	int K = x->K, N = x->N;

	for (int i0 = m0; i0 < m1; i0 += TM) {
		int i1 = imin(i0 + TM, m1);
		for (int j0 = 0; j0 < N; j0 += TN) {
			int j1 = imin(j0 + TN, N);
			float acc[TM][TN] = {{0}};
			for (int k0 = 0; k0 < K; k0 += TK)
				for (int i = i0; i < i1; i++)
					for (int k = k0; k < imin(k0 + TK, K); k++) {
						float av = oracle_fp16_to_f32(
							a[(size_t)i * K + k]);
						for (int j = j0; j < j1; j++)
							acc[i - i0][j - j0] += av *
								oracle_fp16_to_f32(
								b[(size_t)k * N + j]);
					}
			for (int i = i0; i < i1; i++)
				for (int j = j0; j < j1; j++)
					c[(size_t)i * N + j] =
						oracle_f32_to_fp16(acc[i - i0][j - j0]);
		}
	}
}

void oracle_matmul_f16_acc32(const uint16_t *a, const uint16_t *b,
			     uint16_t *c, int M, int K, int N, int n_threads)
{
	struct mm_ctx x = { a, b, c, M, K, N };
	run_rows(mm_f16acc32_rows, &x, M, n_threads);
}

/* ---- Q8: cpu_matmul_q8.c:39-134, x86 scalar loop :124-131.
 * B[K,N] is one flat array of blocks over the linear index k*N + n.
 * Per output element: c += (a * (float)q) * scale, k ascending. ---- */
static void mm_q8_rows(void *p, int m0, int m1)
{
	struct mm_ctx *x = p;
	const float *a = x->a;
	const struct q8blk *blk = x->b;
	float *c = x->c;
	int K = x->K, N = x->N;

	for (int i = m0; i < m1; i++) {
		float *crow = c + (size_t)i * N;
		memset(crow, 0, (size_t)N * sizeof(float));
		for (int k = 0; k < K; k++) {
			float av = a[(size_t)i * K + k];
			size_t lin = (size_t)k * N;
			for (int j = 0; j < N; j++, lin++) {
				const struct q8blk *bb = &blk[lin / ORACLE_Q8_BLOCK];
				crow[j] += av * (float)bb->q[lin % ORACLE_Q8_BLOCK]
					   * bb->d;
			}
		}
	}
}

void oracle_matmul_q8(const float *a, const void *b_blocks, float *c,
		      int M, int K, int N, int n_threads)
{
	struct mm_ctx x = { a, b_blocks, c, M, K, N };
	run_rows(mm_q8_rows, &x, M, n_threads);
}

/* ---- Q8 with W[N,K] (blocks along K, linear index n*K + k). Column n
 * is exactly the reference Q8 kernel with B = W[n,:] as a [K,1] tensor:
 * c[n] += (a[k] * (float)q) * scale, k ascending. ---- */
static void mm_q8_nt_rows(void *p, int m0, int m1)
{
	struct mm_ctx *x = p;
	const float *a = x->a;
	const struct q8blk *blk = x->b;
	float *c = x->c;
	int K = x->K, N = x->N;

	for (int i = m0; i < m1; i++) {
		const float *arow = a + (size_t)i * K;
		for (int j = 0; j < N; j++) {
			float acc = 0.0f;
			size_t lin = (size_t)j * K;
			for (int k = 0; k < K; k++, lin++) {
				const struct q8blk *bb = &blk[lin / ORACLE_Q8_BLOCK];
				acc += arow[k] * (float)bb->q[lin % ORACLE_Q8_BLOCK]
				       * bb->d;
			}
			c[(size_t)i * N + j] = acc;
		}
	}
}

void oracle_matmul_q8_nt(const float *a, const void *w_blocks, float *c,
			 int M, int K, int N, int n_threads)
{
	struct mm_ctx x = { a, w_blocks, c, M, K, N };
	run_rows(mm_q8_nt_rows, &x, M, n_threads);
}

/* ------------------------------------------------------------------ */
/* Transpose: cpu_transpose.c:355-366 (2-D swap of the last two dims,   */
/* a plain element copy).                                               */
/* ------------------------------------------------------------------ */
void oracle_transpose_u16(const uint16_t *src, uint16_t *dst, int R, int C)
{
	for (int r = 0; r < R; r++)
		for (int c = 0; c < C; c++)
			dst[(size_t)c * R + r] = src[(size_t)r * C + c];
}

void oracle_transpose_f32(const float *src, float *dst, int R, int C)
{
	for (int r = 0; r < R; r++)
		for (int c = 0; c < C; c++)
			dst[(size_t)c * R + r] = src[(size_t)r * C + c];
}

/* ------------------------------------------------------------------ */
/* Bias add: out = x + bias[j] over the last dim                        */
/* (cpu_elementwise.c:28-63 + add_f32_scalar; cpu_add_bf16.c:62-63,     */
/* 86-98; cpu_add_f16.c:87-95: convert, add in f32, round once).         */
/* ------------------------------------------------------------------ */
void oracle_bias_add_f32(const float *x, const float *bias, float *out,
			 int rows, int N)
{
	for (int r = 0; r < rows; r++)
		for (int j = 0; j < N; j++)
			out[(size_t)r * N + j] = x[(size_t)r * N + j] + bias[j];
}

void oracle_bias_add_bf16(const uint16_t *x, const uint16_t *bias,
			  uint16_t *out, int rows, int N)
{
	for (int r = 0; r < rows; r++)
		for (int j = 0; j < N; j++)
			out[(size_t)r * N + j] = oracle_f32_to_bf16(
				oracle_bf16_to_f32(x[(size_t)r * N + j]) +
				oracle_bf16_to_f32(bias[j]));
}

void oracle_bias_add_f16(const uint16_t *x, const uint16_t *bias,
			 uint16_t *out, int rows, int N)
{
	for (int r = 0; r < rows; r++)
		for (int j = 0; j < N; j++)
			out[(size_t)r * N + j] = oracle_f32_to_fp16(
				oracle_fp16_to_f32(x[(size_t)r * N + j]) +
				oracle_fp16_to_f32(bias[j]));
}

/* ------------------------------------------------------------------ */
/* tanh-GELU: cpu_gelu.c:23-38, cpu_gelu_bf16.c:62-64,                  */
/* cpu_gelu_f16.c:52-54. Same operation order as the reference:          */
/* inner = c0 * (x + ((c1*x)*x)*x); out = (0.5*x) * (1 + tanhf(inner)). */
/* ------------------------------------------------------------------ */
static inline float gelu_tanh(float x)
{
	float cube = 0.044715f * x * x * x;
	float inner = 0.7978845608f * (x + cube);
	return 0.5f * x * (1.0f + tanhf(inner));
}

void oracle_gelu_f32(const float *x, float *out, int n)
{
	for (int i = 0; i < n; i++)
		out[i] = gelu_tanh(x[i]);
}

void oracle_gelu_bf16(const uint16_t *x, uint16_t *out, int n)
{
	for (int i = 0; i < n; i++)
		out[i] = oracle_f32_to_bf16(gelu_tanh(oracle_bf16_to_f32(x[i])));
}

void oracle_gelu_f16(const uint16_t *x, uint16_t *out, int n)
{
	for (int i = 0; i < n; i++)
		out[i] = oracle_f32_to_fp16(gelu_tanh(oracle_fp16_to_f32(x[i])));
}

/* ------------------------------------------------------------------ */
/* Batched bf16: the reference has no batched matmul (the kernels use  */
/* only the last two dims, cpu_matmul_bf16.c:213-236), so attention's   */
/* QK^T / PV are restated as the 2-D kernel per slice, with a per-slice */
/* transpose for B stored [N,K] (gh_transpose + gh_matmul).             */
/* ------------------------------------------------------------------ */
void oracle_matmul_bf16_batched(const uint16_t *a, const uint16_t *b,
				uint16_t *c, int batch, int M, int K, int N,
				int b_nt, int n_threads)
{
	uint16_t *tmp = NULL;

	if (b_nt) {
		tmp = malloc((size_t)K * N * sizeof(uint16_t));
		if (!tmp)
			return;
	}
	for (int s = 0; s < batch; s++) {
		const uint16_t *as = a + (size_t)s * M * K;
		const uint16_t *bs = b + (size_t)s * K * N;
		uint16_t *cs = c + (size_t)s * M * N;
		if (b_nt) {
			oracle_transpose_u16(bs, tmp, N, K);
			bs = tmp;
		}
		oracle_matmul_bf16(as, bs, cs, M, K, N, n_threads);
	}
	free(tmp);
}

/* ------------------------------------------------------------------ */
/* SDPA: src/backend/cpu/kernels/cpu_sdpa.c:49-159 (x86 scalar branch)  */
/* and :216-288. softmax(Q K^T / sqrt(hd) + mask) V per query row with  */
/* the reference's online softmax: one key at a time, running max and   */
/* sum, the output rescaled by expf(old_max - new_max) whenever the max */
/* grows. Q [BH, Sq, D], K and V [BH, Sk, D], mask [Sq, Sk] (shared by  */
/* all heads) or NULL, out [BH, Sq, D]. Rows split across threads.      */
/* ------------------------------------------------------------------ */
struct sdpa_ctx {
	const float *q, *k, *v, *mask;
	float *out;
	int Sq, Sk, D;
	float scale;
};

static void sdpa_row(const float *q, const float *K, const float *V, const float *mrow,
		     float *out, int Sk, int D, float scale)
{
	float row_max = -FLT_MAX;
	float row_sum = 0.0f;

	memset(out, 0, (size_t)D * sizeof(float));
	for (int j = 0; j < Sk; j++) {
		const float *kj = K + (size_t)j * D;
		float score = 0.0f;
		for (int d = 0; d < D; d++)
			score += q[d] * kj[d];
		score *= scale;
		if (mrow)
			score += mrow[j];
		if (score > row_max) {
			float correction = expf(row_max - score);
			row_sum *= correction;
			for (int d = 0; d < D; d++)
				out[d] *= correction;
			row_max = score;
		}
		float w = expf(score - row_max);
		const float *vj = V + (size_t)j * D;
		for (int d = 0; d < D; d++)
			out[d] += w * vj[d];
		row_sum += w;
	}
	if (row_sum > 0.0f) {
		float inv_sum = 1.0f / row_sum;
		for (int d = 0; d < D; d++)
			out[d] *= inv_sum;
	}
}

static void sdpa_rows(void *p, int r0, int r1)
{
	struct sdpa_ctx *x = p;
	for (int idx = r0; idx < r1; idx++) {
		int bh = idx / x->Sq, i = idx % x->Sq;
		const float *q = x->q + ((size_t)bh * x->Sq + i) * x->D;
		const float *k = x->k + (size_t)bh * x->Sk * x->D;
		const float *v = x->v + (size_t)bh * x->Sk * x->D;
		const float *m = x->mask ? x->mask + (size_t)i * x->Sk : NULL;
		sdpa_row(q, k, v, m, x->out + ((size_t)bh * x->Sq + i) * x->D, x->Sk, x->D, x->scale);
	}
}

void oracle_sdpa_f32(const float *q, const float *k, const float *v, const float *mask,
		     float *out, int BH, int Sq, int Sk, int D, int n_threads)
{
	struct sdpa_ctx x = { q, k, v, mask, out, Sq, Sk, D, 1.0f / sqrtf((float)D) };
	run_rows(sdpa_rows, &x, BH * Sq, n_threads);
}

/* ------------------------------------------------------------------ */
/* LayerNorm: cpu_layernorm.c:28-55 (layernorm_row_scalar, the x86      */
/* build without AVX2), cpu_layernorm_bf16.c:88-115 and                 */
/* cpu_layernorm_f16.c:99-127 (16-bit in/out, f32 arithmetic). Sums run */
/* left to right in f32; mean = sum / cols; inv_std =                   */
/* 1 / sqrtf(var_sum / cols + 1e-5); out = (x - mean) * inv_std, then   */
/* * gamma, then + beta, each rounded. Rows split across threads.       */
/* ------------------------------------------------------------------ */
#define ORACLE_LN_EPS 1e-5f

struct ln_ctx {
	const void *x, *gamma, *beta;
	void *out;
	int cols, kind; /* 0 f32, 1 bf16, 2 f16 */
};

static float ln_get(const void *p, int kind, size_t i)
{
	if (kind == 0)
		return ((const float *)p)[i];
	if (kind == 1)
		return oracle_bf16_to_f32(((const uint16_t *)p)[i]);
	return oracle_fp16_to_f32(((const uint16_t *)p)[i]);
}

static void ln_rows(void *p, int r0, int r1)
{
	struct ln_ctx *c = p;
	const int n = c->cols;
	for (int r = r0; r < r1; r++) {
		const size_t base = (size_t)r * n;
		float sum = 0.0f;
		for (int j = 0; j < n; j++)
			sum += ln_get(c->x, c->kind, base + j);
		float mean = sum / (float)n;
		float var_sum = 0.0f;
		for (int j = 0; j < n; j++) {
			float d = ln_get(c->x, c->kind, base + j) - mean;
			var_sum += d * d;
		}
		float inv_std = 1.0f / sqrtf(var_sum / (float)n + ORACLE_LN_EPS);
		for (int j = 0; j < n; j++) {
			float val = (ln_get(c->x, c->kind, base + j) - mean) * inv_std;
			if (c->gamma)
				val *= ln_get(c->gamma, c->kind, j);
			if (c->beta)
				val += ln_get(c->beta, c->kind, j);
			if (c->kind == 0)
				((float *)c->out)[base + j] = val;
			else if (c->kind == 1)
				((uint16_t *)c->out)[base + j] = oracle_f32_to_bf16(val);
			else
				((uint16_t *)c->out)[base + j] = oracle_f32_to_fp16(val);
		}
	}
}

void oracle_layernorm_f32(const float *x, const float *gamma, const float *beta, float *out,
			  int rows, int cols, int n_threads)
{
	struct ln_ctx c = { x, gamma, beta, out, cols, 0 };
	run_rows(ln_rows, &c, rows, n_threads);
}

void oracle_layernorm_bf16(const uint16_t *x, const uint16_t *gamma, const uint16_t *beta,
			   uint16_t *out, int rows, int cols, int n_threads)
{
	struct ln_ctx c = { x, gamma, beta, out, cols, 1 };
	run_rows(ln_rows, &c, rows, n_threads);
}

void oracle_layernorm_f16(const uint16_t *x, const uint16_t *gamma, const uint16_t *beta,
			  uint16_t *out, int rows, int cols, int n_threads)
{
	struct ln_ctx c = { x, gamma, beta, out, cols, 2 };
	run_rows(ln_rows, &c, rows, n_threads);
}

/* ------------------------------------------------------------------ */
/* RoPE: cpu_rope.c:88-104 and the 16-bit twins cpu_rope_bf16.c:100-121 */
/* and cpu_rope_f16.c:100-121. x [batch, seq, heads, hd]; the pair      */
/* (2d, 2d+1) of every head at position s turns by the angle of         */
/* cos/sin[s][d]: y0 = x0*c - x1*s, y1 = x0*s + x1*c, each product      */
/* rounded (no contraction), 16-bit inputs widened and the results      */
/* rounded once.                                                        */
/* ------------------------------------------------------------------ */
static void rope_any(const void *x, const float *cos_t, const float *sin_t, void *y, int batch,
		     int seq, int heads, int hd, int kind)
{
	const int half = hd / 2;
	for (int b = 0; b < batch; b++)
		for (int s = 0; s < seq; s++) {
			const float *cs = cos_t + (size_t)s * half;
			const float *sn = sin_t + (size_t)s * half;
			for (int h = 0; h < heads; h++) {
				const size_t off = (((size_t)b * seq + s) * heads + h) * hd;
				for (int d = 0; d < half; d++) {
					float x0 = ln_get(x, kind, off + 2 * d);
					float x1 = ln_get(x, kind, off + 2 * d + 1);
					float y0 = x0 * cs[d] - x1 * sn[d];
					float y1 = x0 * sn[d] + x1 * cs[d];
					if (kind == 0) {
						((float *)y)[off + 2 * d] = y0;
						((float *)y)[off + 2 * d + 1] = y1;
					} else if (kind == 1) {
						((uint16_t *)y)[off + 2 * d] = oracle_f32_to_bf16(y0);
						((uint16_t *)y)[off + 2 * d + 1] = oracle_f32_to_bf16(y1);
					} else {
						((uint16_t *)y)[off + 2 * d] = oracle_f32_to_fp16(y0);
						((uint16_t *)y)[off + 2 * d + 1] = oracle_f32_to_fp16(y1);
					}
				}
			}
		}
}

void oracle_rope_f32(const float *x, const float *cos_t, const float *sin_t, float *y,
		     int batch, int seq, int heads, int hd)
{
	rope_any(x, cos_t, sin_t, y, batch, seq, heads, hd, 0);
}

void oracle_rope_bf16(const uint16_t *x, const float *cos_t, const float *sin_t, uint16_t *y,
		      int batch, int seq, int heads, int hd)
{
	rope_any(x, cos_t, sin_t, y, batch, seq, heads, hd, 1);
}

void oracle_rope_f16(const uint16_t *x, const float *cos_t, const float *sin_t, uint16_t *y,
		     int batch, int seq, int heads, int hd)
{
	rope_any(x, cos_t, sin_t, y, batch, seq, heads, hd, 2);
}

/* ------------------------------------------------------------------ */
/* Conv2D, NHWC x OHWI: cpu_conv2d.c:46-88 (im2col_nhwc_f32), :98-128   */
/* (col x W^T, out[j] zeroed then out[j] += col[k]*w[j][k] for k in     */
/* order), :296-435 (groups, params); the 16-bit twins                  */
/* cpu_conv2d_bf16.c:42-80, :179-213 and cpu_conv2d_f16.c (scalar path)  */
/* accumulate the same products in f32 and round the output once.       */
/* ------------------------------------------------------------------ */
struct conv_ctx {
	const void *x, *w;
	void *y;
	int kind; /* 0 f32, 1 bf16, 2 f16 */
	int N, H, W, C, OC, KH, KW, stride, ph, pw, groups, OH, OW;
};

static void conv_rows(void *p, int r0, int r1)
{
	const struct conv_ctx *c = p;
	const int cpg_in = c->C / c->groups, cpg_out = c->OC / c->groups;
	const int K = cpg_in * c->KH * c->KW;
	float *col = malloc((size_t)K * sizeof(float));
	float *acc = malloc((size_t)cpg_out * sizeof(float));
	if (!col || !acc) {
		free(col);
		free(acc);
		return;
	}
	for (int r = r0; r < r1; r++) { /* r = (n * OH + oh) * OW + ow */
		const int ow = r % c->OW, oh = (r / c->OW) % c->OH, n = r / (c->OW * c->OH);
		for (int g = 0; g < c->groups; g++) {
			/* im2col row: taps (kh, kw), group channels innermost */
			for (int kh = 0; kh < c->KH; kh++) {
				const int ih = oh * c->stride + kh - c->ph;
				for (int kw = 0; kw < c->KW; kw++) {
					const int iw = ow * c->stride + kw - c->pw;
					float *d = col + ((size_t)kh * c->KW + kw) * cpg_in;
					const int in = (unsigned)ih < (unsigned)c->H && (unsigned)iw < (unsigned)c->W;
					for (int ic = 0; ic < cpg_in; ic++)
						d[ic] = in ? ln_get(c->x, c->kind,
								    (((size_t)n * c->H + ih) * c->W + iw) * c->C +
									    (size_t)g * cpg_in + ic)
							   : 0.0f;
				}
			}
			const size_t wg = (size_t)g * cpg_out * K;
			for (int j = 0; j < cpg_out; j++)
				acc[j] = 0.0f;
			for (int k = 0; k < K; k++) {
				const float cik = col[k];
				for (int j = 0; j < cpg_out; j++)
					acc[j] += cik * ln_get(c->w, c->kind, wg + (size_t)j * K + k);
			}
			const size_t ob = (size_t)r * c->OC + (size_t)g * cpg_out;
			for (int j = 0; j < cpg_out; j++) {
				if (c->kind == 0)
					((float *)c->y)[ob + j] = acc[j];
				else if (c->kind == 1)
					((uint16_t *)c->y)[ob + j] = oracle_f32_to_bf16(acc[j]);
				else
					((uint16_t *)c->y)[ob + j] = oracle_f32_to_fp16(acc[j]);
			}
		}
	}
	free(col);
	free(acc);
}

static void conv_any(const void *x, const void *w, void *y, int kind, int N, int H, int W, int C,
		     int OC, int KH, int KW, int stride, int ph, int pw, int groups, int OH, int OW,
		     int n_threads)
{
	struct conv_ctx c = { x, w, y, kind, N, H, W, C, OC, KH, KW, stride, ph, pw, groups, OH, OW };
	run_rows(conv_rows, &c, N * OH * OW, n_threads);
}

void oracle_conv2d_f32(const float *x, const float *w, float *y, int N, int H, int W, int C,
		       int OC, int KH, int KW, int stride, int ph, int pw, int groups, int OH, int OW,
		       int n_threads)
{
	conv_any(x, w, y, 0, N, H, W, C, OC, KH, KW, stride, ph, pw, groups, OH, OW, n_threads);
}

void oracle_conv2d_bf16(const uint16_t *x, const uint16_t *w, uint16_t *y, int N, int H, int W,
			int C, int OC, int KH, int KW, int stride, int ph, int pw, int groups, int OH,
			int OW, int n_threads)
{
	conv_any(x, w, y, 1, N, H, W, C, OC, KH, KW, stride, ph, pw, groups, OH, OW, n_threads);
}

void oracle_conv2d_f16(const uint16_t *x, const uint16_t *w, uint16_t *y, int N, int H, int W,
		       int C, int OC, int KH, int KW, int stride, int ph, int pw, int groups, int OH,
		       int OW, int n_threads)
{
	conv_any(x, w, y, 2, N, H, W, C, OC, KH, KW, stride, ph, pw, groups, OH, OW, n_threads);
}

/* ------------------------------------------------------------------ */
/* ConvTranspose2D, NHWC x OHWI (cpu_conv_transpose2d.c:55-131): per    */
/* output pixel the channels start at 0; for each tap (kh, kw) whose    */
/* input pixel ih = (oh + pad - kh) / stride divides exactly and lies   */
/* inside, out[co] += dot over input channels in order.                 */
/* ------------------------------------------------------------------ */
struct convt_ctx {
	const float *x, *w;
	float *y;
	int N, H, W, C, OC, KH, KW, stride, pad, OH, OW;
};

static void convt_rows(void *p, int r0, int r1)
{
	const struct convt_ctx *c = p;
	const size_t kk = (size_t)c->KH * c->KW * c->C;
	for (int row = r0; row < r1; row++) { /* row = n * OH + oh */
		const int n = row / c->OH, oh = row % c->OH;
		for (int ow = 0; ow < c->OW; ow++) {
			float *out = c->y + (((size_t)n * c->OH + oh) * c->OW + ow) * c->OC;
			for (int co = 0; co < c->OC; co++)
				out[co] = 0.0f;
			for (int kh = 0; kh < c->KH; kh++) {
				const int ohf = oh + c->pad - kh;
				if (ohf < 0 || ohf % c->stride != 0)
					continue;
				const int ih = ohf / c->stride;
				if (ih >= c->H)
					continue;
				for (int kw = 0; kw < c->KW; kw++) {
					const int owf = ow + c->pad - kw;
					if (owf < 0 || owf % c->stride != 0)
						continue;
					const int iw = owf / c->stride;
					if (iw >= c->W)
						continue;
					const float *in = c->x + (((size_t)n * c->H + ih) * c->W + iw) * c->C;
					for (int co = 0; co < c->OC; co++) {
						const float *wp = c->w + (size_t)co * kk + ((size_t)kh * c->KW + kw) * c->C;
						float dot = 0.0f;
						for (int ci = 0; ci < c->C; ci++)
							dot += in[ci] * wp[ci];
						out[co] += dot;
					}
				}
			}
		}
	}
}

void oracle_conv_transpose2d_f32(const float *x, const float *w, float *y, int N, int H, int W,
				 int C, int OC, int KH, int KW, int stride, int pad, int n_threads)
{
	struct convt_ctx c = { x, w, y, N, H, W, C, OC, KH, KW, stride, pad,
			       (H - 1) * stride - 2 * pad + KH, (W - 1) * stride - 2 * pad + KW };
	run_rows(convt_rows, &c, N * c.OH, n_threads);
}

/* ------------------------------------------------------------------ */
/* MaxPool2D, NHWC (cpu_maxpool2d.c:68-108): start from the window's    */
/* first tap, then take a tap only when it is greater; taps past the    */
/* image are skipped. OH = (H - kernel) / stride + 1.                   */
/* ------------------------------------------------------------------ */
void oracle_maxpool2d_f32(const float *x, float *y, int N, int H, int W, int C, int kernel,
			  int stride)
{
	const int OH = (H - kernel) / stride + 1, OW = (W - kernel) / stride + 1;
	for (int n = 0; n < N; n++)
		for (int oh = 0; oh < OH; oh++)
			for (int ow = 0; ow < OW; ow++) {
				float *out = y + (((size_t)n * OH + oh) * OW + ow) * C;
				const int ih0 = oh * stride, iw0 = ow * stride;
				const float *first = x + (((size_t)n * H + ih0) * W + iw0) * C;
				for (int c = 0; c < C; c++)
					out[c] = first[c];
				for (int kh = 0; kh < kernel; kh++)
					for (int kw = 0; kw < kernel; kw++) {
						const int ih = ih0 + kh, iw = iw0 + kw;
						if ((kh == 0 && kw == 0) || ih >= H || iw >= W)
							continue;
						const float *in = x + (((size_t)n * H + ih) * W + iw) * C;
						for (int c = 0; c < C; c++)
							if (in[c] > out[c])
								out[c] = in[c];
					}
			}
}
