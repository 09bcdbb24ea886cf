/*
 * sam3_hip_ops.c - C11 host side of the HIP matmul path: argument and
 * dtype checks, node-level kernels, the per-node dispatcher and the
 * device helpers exported through include/sam3_hip.h.
 *
 * Error behaviour follows the reference CPU path (sam3.c):
 *   - node kernels: NULL tensors, wrong dtypes, K mismatch and output size
 *     mismatch -> SAM3_EINVAL (src/backend/cpu/kernels/cpu_matmul.c:
 *     178-229, cpu_matmul_q8.c:168-213);
 *   - dispatcher: mixed dtypes other than F32 x Q8_0 -> SAM3_EDTYPE, an
 *     (op, dtype) without a kernel -> SAM3_EDTYPE
 *     (src/backend/cpu/cpu_dispatch.c:591-686);
 *   - HIP failures -> SAM3_EBACKEND, device out of memory -> SAM3_ENOMEM.
 * Nothing here aborts; the message of the last failure is kept per thread
 * (sam3_hip_last_error) and printed to stderr unless SAM3_HIP_QUIET is set.
 */
#include "sam3_hip.h"
#include "sam3_hip_internal.h"
#include "s3k.h"

#include <hip/hip_runtime_api.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <stdint.h>
#include <string.h>

static _Thread_local char g_last_error[320];

void s3h_error(const char *fmt, ...)
{
	va_list ap;
	va_start(ap, fmt);
	vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
	va_end(ap);
	if (!s3h_settings()->quiet)
		fprintf(stderr, "[sam3_hip] %s\n", g_last_error);
}

const char *sam3_hip_last_error(void)
{
	return g_last_error;
}

enum sam3_error s3h_hip(int e, const char *what)
{
	if (e == hipSuccess)
		return SAM3_OK;
	s3h_error("%s: %s", what, hipGetErrorString((hipError_t)e));
	return e == hipErrorOutOfMemory ? SAM3_ENOMEM : SAM3_EBACKEND;
}

/* Scratch blocks reused in stream order. A freed block goes back to a
 * free list tagged with the device and the stream of its last use; a
 * later request on that same stream may take it at once, because every
 * kernel that used it was enqueued on that stream before the new user.
 * Blocks are never handed to another stream. Requests take the smallest
 * free block that fits and is at most twice the request (or 4 MiB
 * larger); otherwise a new block is allocated with hipMalloc, after
 * returning the idle blocks of the device to the runtime if the first
 * attempt runs out of memory. This replaces stream-ordered
 * hipMallocAsync / hipFreeAsync pairs, each of which left the GPU idle
 * for about 5 us between the kernels around it. */
struct s3h_blk {
	void *p;
	size_t n;
	void *stream;
	int dev;
	int busy;
};
static struct s3h_blk *s3h_blks;
static int s3h_nblks, s3h_capblks;
/* The idle blocks (indices into s3h_blks), which is all a request scans,
 * and an open-addressing index block address -> slot + 1 for frees: a
 * backend keeps hundreds of blocks busy (its resident weights), so
 * neither may walk the whole table. The index is rebuilt after the table
 * changes order (a trim). */
static int *s3h_idle, s3h_nidle, s3h_capidle;
static int *s3h_bix;
static size_t s3h_bix_cap;
static int s3h_bix_dirty;
static pthread_mutex_t s3h_blk_lock = PTHREAD_MUTEX_INITIALIZER;

static size_t blk_hash(const void *p)
{
	uint64_t x = (uint64_t)(uintptr_t)p;
	x ^= x >> 33;
	x *= 0xff51afd7ed558ccdULL;
	x ^= x >> 33;
	return (size_t)x;
}

static void bix_put(int slot)
{
	size_t k = blk_hash(s3h_blks[slot].p) & (s3h_bix_cap - 1);
	while (s3h_bix[k])
		k = (k + 1) & (s3h_bix_cap - 1);
	s3h_bix[k] = slot + 1;
}

static int bix_rebuild(void)
{
	size_t cap = 64;
	while (cap < 4 * (size_t)s3h_nblks)
		cap <<= 1;
	if (cap != s3h_bix_cap) {
		int *ix = realloc(s3h_bix, cap * sizeof(*ix));
		if (!ix)
			return 0;
		s3h_bix = ix;
		s3h_bix_cap = cap;
	}
	memset(s3h_bix, 0, s3h_bix_cap * sizeof(*s3h_bix));
	for (int i = 0; i < s3h_nblks; i++)
		bix_put(i);
	s3h_bix_dirty = 0;
	return 1;
}

/* Slot of block p, or -1. Called with the lock held. */
static int blk_slot(const void *p)
{
	if ((s3h_bix_dirty || 2 * (size_t)s3h_nblks >= s3h_bix_cap) && !bix_rebuild()) {
		for (int i = 0; i < s3h_nblks; i++)
			if (s3h_blks[i].p == p)
				return i;
		return -1;
	}
	size_t k = blk_hash(p) & (s3h_bix_cap - 1);
	while (s3h_bix[k]) {
		const int i = s3h_bix[k] - 1;
		if (s3h_blks[i].p == p)
			return i;
		k = (k + 1) & (s3h_bix_cap - 1);
	}
	return -1;
}

static int idle_push(int slot)
{
	if (s3h_nidle == s3h_capidle) {
		const int cap = s3h_capidle ? 2 * s3h_capidle : 64;
		int *t = realloc(s3h_idle, (size_t)cap * sizeof(*t));
		if (!t)
			return 0;
		s3h_idle = t;
		s3h_capidle = cap;
	}
	s3h_idle[s3h_nidle++] = slot;
	return 1;
}

static size_t scratch_round(size_t n)
{
	const size_t g = n > ((size_t)1 << 20) ? ((size_t)1 << 20) : 256;
	return n ? (n + g - 1) / g * g : g;
}

/* hipFree every idle block of device dev (all streams when stream_only
 * is 0, else only those of `stream`), after the work using them is done.
 * Called with the lock held. */
static void scratch_trim_locked(int dev, int stream_only, void *stream)
{
	int synced = 0;
	for (int i = s3h_nblks - 1; i >= 0; i--) {
		struct s3h_blk *b = &s3h_blks[i];
		if (b->busy || b->dev != dev || (stream_only && b->stream != stream))
			continue;
		if (!synced) {
			if (stream_only)
				(void)hipStreamSynchronize((hipStream_t)stream);
			else
				(void)hipDeviceSynchronize();
			synced = 1;
		}
		(void)hipFree(b->p);
		s3h_blks[i] = s3h_blks[--s3h_nblks];
	}
	/* slots moved: rebuild the idle list and the address index */
	s3h_nidle = 0;
	for (int i = 0; i < s3h_nblks; i++)
		if (!s3h_blks[i].busy)
			(void)idle_push(i); /* the list only shrank: no allocation */
	s3h_bix_dirty = 1;
}

enum sam3_error s3h_scratch_alloc(void **p, size_t nbytes, void *stream)
{
	int dev = 0;
	(void)hipGetDevice(&dev);
	const size_t need = scratch_round(nbytes);
	const size_t most = need * 2 > need + ((size_t)4 << 20) ? need * 2 : need + ((size_t)4 << 20);
	*p = NULL;
	pthread_mutex_lock(&s3h_blk_lock);
	int best = -1;
	for (int j = 0; j < s3h_nidle; j++) {
		const struct s3h_blk *b = &s3h_blks[s3h_idle[j]];
		if (b->dev == dev && b->stream == stream && b->n >= need && b->n <= most &&
		    (best < 0 || b->n < s3h_blks[s3h_idle[best]].n))
			best = j;
	}
	if (best >= 0) {
		const int slot = s3h_idle[best];
		s3h_idle[best] = s3h_idle[--s3h_nidle];
		s3h_blks[slot].busy = 1;
		*p = s3h_blks[slot].p;
		pthread_mutex_unlock(&s3h_blk_lock);
		return SAM3_OK;
	}
	if (s3h_nblks == s3h_capblks) {
		const int cap = s3h_capblks ? s3h_capblks * 2 : 64;
		struct s3h_blk *t = realloc(s3h_blks, (size_t)cap * sizeof(*t));
		if (!t) {
			pthread_mutex_unlock(&s3h_blk_lock);
			s3h_error("scratch: out of host memory for the block table");
			return SAM3_ENOMEM;
		}
		s3h_blks = t;
		s3h_capblks = cap;
	}
	/* room in the idle list for this block's later free */
	if (s3h_capidle < s3h_nblks + 1) {
		const int cap = 2 * (s3h_nblks + 1);
		int *t = realloc(s3h_idle, (size_t)cap * sizeof(*t));
		if (!t) {
			pthread_mutex_unlock(&s3h_blk_lock);
			s3h_error("scratch: out of host memory for the idle list");
			return SAM3_ENOMEM;
		}
		s3h_idle = t;
		s3h_capidle = cap;
	}
	void *q = NULL;
	hipError_t e = hipMalloc(&q, need);
	if (e == hipErrorOutOfMemory) {
		(void)hipGetLastError();
		scratch_trim_locked(dev, 0, NULL);
		e = hipMalloc(&q, need);
	}
	if (e != hipSuccess) {
		pthread_mutex_unlock(&s3h_blk_lock);
		return s3h_hip(e, "scratch");
	}
	s3h_blks[s3h_nblks++] = (struct s3h_blk){q, need, stream, dev, 1};
	if (!s3h_bix_dirty && 2 * (size_t)s3h_nblks < s3h_bix_cap)
		bix_put(s3h_nblks - 1);
	else
		s3h_bix_dirty = 1;
	*p = q;
	pthread_mutex_unlock(&s3h_blk_lock);
	return SAM3_OK;
}

enum sam3_error s3h_scratch_free(void *p, void *stream)
{
	if (!p)
		return SAM3_OK;
	pthread_mutex_lock(&s3h_blk_lock);
	const int i = blk_slot(p);
	if (i >= 0) {
		if (s3h_blks[i].busy) {
			s3h_blks[i].busy = 0;
			s3h_blks[i].stream = stream; /* its last use was enqueued here */
			(void)idle_push(i); /* room was reserved when the block was made */
		}
		pthread_mutex_unlock(&s3h_blk_lock);
		return SAM3_OK;
	}
	pthread_mutex_unlock(&s3h_blk_lock);
	s3h_error("scratch: free of %p, which is not a scratch block", p);
	return SAM3_EINVAL;
}

void s3h_scratch_release(void *stream)
{
	int dev = 0;
	(void)hipGetDevice(&dev);
	pthread_mutex_lock(&s3h_blk_lock);
	scratch_trim_locked(dev, 1, stream);
	pthread_mutex_unlock(&s3h_blk_lock);
}

/* ------------------------------------------------------------------ */
/* dtype helpers                                                        */
/* ------------------------------------------------------------------ */
size_t s3h_dtype_size(int dt)
{
	switch (dt) {
	case SAM3_DTYPE_F32:
	case SAM3_DTYPE_I32:
		return 4;
	case SAM3_DTYPE_F16:
	case SAM3_DTYPE_BF16:
		return 2;
	case SAM3_DTYPE_I8:
		return 1;
	default:
		return 0; /* Q8_0 has no element size (src/core/tensor.c:40) */
	}
}

long long s3h_nelems(const struct sam3_tensor *t)
{
	long long n = 1;
	for (int i = 0; i < t->n_dims; i++)
		n *= t->dims[i];
	return n;
}

size_t s3h_tensor_bytes(const struct sam3_tensor *t)
{
	long long n = s3h_nelems(t);
	if (t->dtype == SAM3_DTYPE_Q8_0)
		return (size_t)((n + 31) / 32) * 36;
	return (size_t)n * s3h_dtype_size(t->dtype);
}

static int is_float_dtype(int dt)
{
	return dt == SAM3_DTYPE_F32 || dt == SAM3_DTYPE_F16 || dt == SAM3_DTYPE_BF16;
}

/* ------------------------------------------------------------------ */
/* Plain-pointer matmul                                                 */
/* ------------------------------------------------------------------ */
static enum sam3_error check_kinds(int a_dt, int b_dt, int c_dt)
{
	if (b_dt == SAM3_DTYPE_Q8_0) {
		/* the Q8 kernels write F32, as cpu_matmul_q8.c:181-185 does */
		if (!is_float_dtype(a_dt) || c_dt != SAM3_DTYPE_F32) {
			s3h_error("matmul: Q8_0 needs F32/F16/BF16 activations and an F32 "
				  "output (a=%d c=%d)", a_dt, c_dt);
			return SAM3_EDTYPE;
		}
		return SAM3_OK;
	}
	if (!is_float_dtype(a_dt) || a_dt != b_dt ||
	    (c_dt != a_dt && c_dt != SAM3_DTYPE_F32)) {
		s3h_error("matmul: unsupported dtypes a=%d b=%d c=%d", a_dt, b_dt, c_dt);
		return SAM3_EDTYPE;
	}
	return SAM3_OK;
}

static void fill_gemm(struct s3k_gemm *g, int a_dt, const void *a, int b_dt, const void *b,
		      int c_dt, void *c, int M, int N, int K, const void *bias, int flags)
{
	memset(g, 0, sizeof(*g));
	g->a = a;
	g->b = b;
	g->c = c;
	g->bias = bias;
	g->M = M;
	g->N = N;
	g->K = K;
	g->lda = K;
	g->ldb = (flags & SAM3_HIP_B_NT) ? K : N;
	g->ldc = N;
	g->batch = 1;
	g->a_kind = a_dt;
	g->b_kind = b_dt;
	g->c_kind = c_dt;
	g->flags = flags & (S3K_EPI_BIAS | S3K_EPI_GELU | S3K_B_NT);
}

/* f32 or bf16 activations of a kernel that rounds them to f16 (the Q8
 * GEMMs and GEMVs, and the f16 GEMM on unpacked Q8 weights): copied row
 * by row to f16 with a power-of-two factor per row (s3k_cast_f16_rows),
 * so rows outside the f16 range (|a| >= 2^15, or all below 2^-10) are
 * scaled into it instead of turning into inf or losing their bits; g
 * then reads the copy and multiplies row m of its result by rs[m] before
 * the bias (S3K_EPI_ROWSCALE), which undoes the factor exactly. Slices
 * sharing their activations (batch stride 0) are copied once. *tmp gets
 * the scratch block, the caller's to free. */
static size_t a_rows_f16_bytes(const struct s3k_gemm *g, size_t *a_bytes)
{
	const int nb = g->batch > 1 && g->stride_a == 0 ? 1 : g->batch;
	*a_bytes = ((size_t)nb * g->M * g->K * 2 + 255) & ~(size_t)255;
	return *a_bytes + (size_t)nb * g->M * 4;
}

/* The copy into buf (a_rows_f16_bytes of g, 16-byte aligned). */
static enum sam3_error a_rows_f16_into(struct s3k_gemm *g, void *buf, void *stream)
{
	const int shared = g->batch > 1 && g->stride_a == 0;
	const int nb = shared ? 1 : g->batch;
	size_t a_bytes;
	(void)a_rows_f16_bytes(g, &a_bytes);
	float *rs = (float *)((char *)buf + a_bytes);
	enum sam3_error err = s3h_hip(s3k_cast_f16_rows(g->a_kind, g->a, g->lda, g->stride_a, buf, rs,
							nb, g->M, g->K, stream),
				      "matmul activation cast");
	if (err != SAM3_OK)
		return err;
	g->a = buf;
	g->a_kind = S3K_F16;
	g->lda = g->K;
	g->stride_a = shared ? 0 : (long long)g->M * g->K;
	g->rs = rs;
	g->rs_sb = shared ? 0 : g->M;
	g->flags |= S3K_EPI_ROWSCALE;
	return SAM3_OK;
}

static enum sam3_error a_rows_f16(struct s3k_gemm *g, void **tmp, void *stream)
{
	size_t a_bytes;
	*tmp = NULL;
	enum sam3_error err = s3h_scratch_alloc(tmp, a_rows_f16_bytes(g, &a_bytes), stream);
	if (err != SAM3_OK)
		return err;
	return a_rows_f16_into(g, *tmp, stream);
}

/* Whether kernel path `path` of g rounds f32/bf16 activations to f16. */
static int rounds_a_to_f16(const struct s3k_gemm *g, int path)
{
	if (g->a_kind == S3K_F16 || (path != S3K_PATH_MFMA && path != S3K_PATH_SKINNY))
		return 0;
	if (path == S3K_PATH_SKINNY && s3k_skinny_scales_rows(g))
		return 0; /* q8_stream scales the rows itself */
	return g->b_kind == S3K_Q8 || (g->b_kind == S3K_F16 && g->a_kind != S3K_F16);
}

/* g on kernel path `path`, after the row-scaled f16 copy of its
 * activations where that path would round them to f16. */
static enum sam3_error q8_colscale(struct s3k_gemm *g, void **own, void *stream);

static enum sam3_error launch_a_safe(const struct s3k_gemm *g, int path, const char *what,
				     void *stream)
{
	if (g->b_kind == S3K_Q8 && path == S3K_PATH_MFMA &&
	    !(g->flags & (S3K_EPI_COLSCALE | S3K_Q8_WAUTO))) {
		/* the MFMA kernels round q*scale to f16: with the weight-row
		 * factors */
		struct s3k_gemm h = *g;
		void *own = NULL;
		enum sam3_error err = q8_colscale(&h, &own, stream);
		if (err == SAM3_OK)
			err = launch_a_safe(&h, path, what, stream);
		if (own) {
			enum sam3_error ferr = s3h_scratch_free(own, stream);
			if (err == SAM3_OK)
				err = ferr;
		}
		return err;
	}
	if (!rounds_a_to_f16(g, path)) {
		int e = s3k_gemm_launch_path(g, path, stream);
		if (e == hipErrorInvalidValue) {
			s3h_error("%s: path %d cannot run M=%d N=%d K=%d", what, path, g->M, g->N,
				  g->K);
			return SAM3_EINVAL;
		}
		return s3h_hip(e, what);
	}
	struct s3k_gemm h = *g;
	void *tmp = NULL;
	enum sam3_error err = a_rows_f16(&h, &tmp, stream);
	if (err == SAM3_OK) {
		int e = s3k_gemm_launch_path(&h, path, stream);
		if (e == hipErrorInvalidValue) {
			s3h_error("%s: path %d cannot run M=%d N=%d K=%d", what, path, g->M, g->N,
				  g->K);
			err = SAM3_EINVAL;
		} else {
			err = s3h_hip(e, what);
		}
	}
	if (tmp) {
		enum sam3_error ferr = s3h_scratch_free(tmp, stream);
		if (err == SAM3_OK)
			err = ferr;
	}
	return err;
}

/* Q8 layouts the tiled kernels cannot stream (blocks over the [K,N] flat
 * index, or [N,K] rows that split blocks): unpacked, with the weight-row
 * factors, to f16 [N,K] in stream-ordered scratch, and the f16 NT GEMM
 * runs on it with the factors in its epilogue (S3K_EPI_COLSCALE). When
 * the f16 problem would not reach the MFMA GEMM, the generic kernel runs
 * on the Q8_0 blocks instead. */
static enum sam3_error q8_unpacked(struct s3k_gemm *g, void *stream)
{
	const int nt = g->flags & S3K_B_NT;
	const size_t bytes = (size_t)g->N * g->K * 2;
	struct s3k_gemm h = *g;
	h.b_kind = S3K_F16;
	h.ldb = g->K;
	h.flags |= S3K_B_NT;
	if (s3k_gemm_path(&h) != S3K_PATH_MFMA)
		return s3h_hip(s3k_gemm_launch_path(g, S3K_PATH_GENERIC, stream), "matmul_q8 generic");
	void *w16 = NULL;
	enum sam3_error err = s3h_scratch_alloc(&w16, bytes + (size_t)g->N * 4, stream);
	if (err != SAM3_OK)
		return err;
	float *cs = (float *)((char *)w16 + bytes);
	int e = 0;
	if (nt) {
		e = s3k_q8_nk_to_f16_nk(g->b, w16, cs, g->K, g->N, stream);
	} else {
		e = s3k_q8_wfactors(g->b, cs, g->K, g->N, 0, 1, 0, stream);
		if (!e)
			e = s3k_q8_kn_to_f16_nk(g->b, w16, cs, g->K, g->N, stream);
	}
	err = s3h_hip(e, "matmul_q8 unpack");
	if (err == SAM3_OK) {
		h.b = w16;
		h.cs = cs;
		h.cs_sb = 0;
		h.flags |= S3K_EPI_COLSCALE;
		err = launch_a_safe(&h, S3K_PATH_MFMA, "matmul_q8 gemm", stream);
	}
	enum sam3_error ferr = s3h_scratch_free(w16, stream);
	return err != SAM3_OK ? err : ferr;
}

/* A prepared copy of weight w (rows x k source elements of 4 or 2 bytes)
 * in the layout `tag` with pitch k_out: from the backend's cache when it
 * holds one, else made by fn into new scratch, which is kept in the cache
 * when w is a constant weight (*own = 0) or is the caller's to free
 * (*own = 1). */
typedef int (*prep_fn)(const void *w, void *out, int rows, int k, int k_out, int kind,
		       void *stream);
static enum sam3_error prep_weight(const void *w, size_t w_bytes, int tag, int rows, int k, int k_out,
				   size_t out_bytes, int kind, prep_fn fn, void *stream, void **out,
				   int *own)
{
	*own = 0;
	*out = s3h_prep_find(w, tag, rows, k_out);
	if (*out)
		return SAM3_OK;
	enum sam3_error err = s3h_scratch_alloc(out, out_bytes, stream);
	if (err == SAM3_OK)
		err = s3h_hip(fn(w, *out, rows, k, k_out, kind, stream), "weight preparation");
	if (err == SAM3_OK && s3h_prep_cacheable(w, w_bytes)) {
		err = s3h_prep_store(w, tag, rows, k_out, *out, out_bytes);
		*own = err != SAM3_OK;
	} else {
		*own = 1;
	}
	return err;
}

static int prep_split_w(const void *w, void *out, int rows, int k, int k_out, int kind, void *stream)
{
	(void)k_out;
	(void)kind;
	return s3k_split3_bf16((const float *)w, out, rows, k, k, 1, stream);
}

static int prep_conv_w(const void *w, void *out, int rows, int k, int k_out, int kind, void *stream)
{
	return s3k_conv_wprep(kind, w, out, rows, k, k_out, stream);
}

/* f16 [rows, k] followed by the weight-row factors f32 [rows] */
static int prep_q8_f16(const void *w, void *out, int rows, int k, int k_out, int kind, void *stream)
{
	(void)k_out;
	(void)kind;
	return s3k_q8_nk_to_f16_nk(w, out, (float *)((char *)out + (size_t)rows * k * 2), k, rows,
				   stream);
}

static int prep_q8_cs(const void *w, void *out, int rows, int k, int k_out, int kind, void *stream)
{
	(void)k_out;
	(void)kind;
	return s3k_q8_wfactors(w, (float *)out, k, rows, 1, 1, 0, stream);
}

/* The weight-row factors (S3K_EPI_COLSCALE, s3k_q8_wfactors) of g's
 * Q8_0 [N,K] weight for an MFMA kernel that rounds q*scale to f16: from
 * the backend's prepared-weight cache when the weight is constant (made
 * once there), else computed into scratch that *own returns for the
 * caller to free. A batch of distinct weights (stride_b != 0) gets the
 * factors of every slice, cs_sb = N apart. */
/* Whether the MFMA kernel that g (Q8_0 weight) reaches finds the
 * weight-row factors itself (S3K_Q8_WAUTO: gemm_dlq8 / gemm_dlpq on f16
 * activations, or on the f16 copy of f32 / bf16 ones). */
static int q8_wauto_ok(const struct s3k_gemm *g)
{
	return g->b_kind == S3K_Q8 && s3h_settings()->q8_wauto && s3k_dlq8_eligible(g);
}

static enum sam3_error q8_colscale(struct s3k_gemm *g, void **own, void *stream)
{
	*own = NULL;
	if (!(g->flags & S3K_B_NT)) {
		s3h_error("matmul_q8: the MFMA kernels read Q8_0 weights as [N, K] only");
		return SAM3_EINVAL;
	}
	const int nb = g->batch > 1 && g->stride_b != 0 ? g->batch : 1;
	/* factors that would be made for this call alone: the kernel finds
	 * them itself when it can (no pass over the weights first) */
	if (q8_wauto_ok(g) &&
	    (nb > 1 || !s3h_prep_cacheable(g->b, ((size_t)g->N * g->K + 31) / 32 * 36))) {
		g->flags |= S3K_Q8_WAUTO;
		return SAM3_OK;
	}
	void *cs = NULL;
	enum sam3_error err;
	if (nb == 1) {
		const size_t q8_bytes = ((size_t)g->N * g->K + 31) / 32 * 36;
		int mine = 0;
		err = prep_weight(g->b, q8_bytes, S3H_PREP_Q8_CS, g->N, g->K, g->K, (size_t)g->N * 4,
				  S3K_Q8, prep_q8_cs, stream, &cs, &mine);
		if (mine)
			*own = cs;
	} else {
		err = s3h_scratch_alloc(&cs, (size_t)nb * g->N * 4, stream);
		if (err == SAM3_OK) {
			*own = cs;
			err = s3h_hip(s3k_q8_wfactors(g->b, (float *)cs, g->K, g->N, 1, nb, g->stride_b,
						      stream),
				      "matmul_q8 weight factors");
		}
	}
	if (err != SAM3_OK)
		return err;
	g->cs = (const float *)cs;
	g->cs_sb = nb > 1 ? g->N : 0;
	g->flags |= S3K_EPI_COLSCALE;
	return SAM3_OK;
}

/* Q8_0 W [N,K] x f16 A on the MFMA path. The weight is expanded into an
 * f16 [N,K] copy, q*scale formed in f32 and rounded once to f16 (the
 * direct Q8 kernel rounds the scale to f16 and multiplies in f16 at every
 * k-step, one more rounding), and the f16 GEMM runs on it at the dense
 * f16 rate. Inside graph_eval a constant weight is expanded once and
 * kept. Other calls expand per call from M = 3072 on, where the f16 GEMM
 * gains more than the expansion pass costs (kernel times, bf16 A, f32
 * out: fc1 N=4096 K=1024 at M = 3072 46.8 us expanded against 55.1 us
 * direct, at M = 5184 69 against 85; at M = 2048 37.0 direct against
 * 42.5), and keep the direct kernel below, which reads 1.125 bytes per
 * weight and needs no scratch. SAM3_HIP_Q8_EXPAND=0 always keeps the
 * direct kernel, =1 always expands. */
#define S3H_Q8_EXPAND_MIN_M 3072
static enum sam3_error q8_f16_gemm(const struct s3k_gemm *h, void *stream)
{
	const int mode = s3h_settings()->q8_expand;
	const size_t q8_bytes = (size_t)h->N * (h->K / 32) * 36;
	const int layout_ok = (h->flags & S3K_B_NT) && h->K % 32 == 0 && h->batch == 1;
	if (layout_ok && mode != 0 &&
	    (mode == 1 || h->M >= S3H_Q8_EXPAND_MIN_M || s3h_prep_cacheable(h->b, q8_bytes))) {
		void *w16 = NULL;
		int own = 0;
		const size_t wbytes = (size_t)h->N * h->K * 2;
		enum sam3_error err = prep_weight(h->b, q8_bytes, S3H_PREP_Q8_F16, h->N, h->K, h->K,
						  wbytes + (size_t)h->N * 4, S3K_Q8, prep_q8_f16,
						  stream, &w16, &own);
		if (err == SAM3_OK) {
			struct s3k_gemm e = *h;
			e.b = w16;
			e.b_kind = S3K_F16;
			e.ldb = h->K;
			e.cs = (const float *)((const char *)w16 + wbytes);
			e.cs_sb = 0;
			e.flags |= S3K_EPI_COLSCALE;
			err = s3h_hip(s3k_gemm_launch_path(&e, S3K_PATH_MFMA, stream), "matmul_q8 f16 gemm");
		}
		if (own && w16) {
			enum sam3_error e2 = s3h_scratch_free(w16, stream);
			if (err == SAM3_OK)
				err = e2;
		}
		return err;
	}
	struct s3k_gemm e = *h;
	void *own = NULL;
	enum sam3_error err = q8_colscale(&e, &own, stream);
	if (err == SAM3_OK)
		err = s3h_hip(s3k_gemm_launch_path(&e, S3K_PATH_MFMA, stream), "matmul_q8 gemm");
	if (own) {
		enum sam3_error e2 = s3h_scratch_free(own, stream);
		if (err == SAM3_OK)
			err = e2;
	}
	return err;
}

/* Whether q8_f16_gemm of h expands the weight for this call alone (not a
 * cached constant weight). */
static int q8_expands_per_call(const struct s3k_gemm *h)
{
	const int mode = s3h_settings()->q8_expand;
	const size_t q8_bytes = (size_t)h->N * (h->K / 32) * 36;
	return (h->flags & S3K_B_NT) && h->K % 32 == 0 && h->batch == 1 && mode != 0 &&
	       (mode == 1 || h->M >= S3H_Q8_EXPAND_MIN_M) && !s3h_prep_cacheable(h->b, q8_bytes) &&
	       !s3h_prep_find(h->b, S3H_PREP_Q8_F16, h->N, h->K);
}

/* f32/bf16 activations times Q8_0 [N,K] weights on the direct-to-LDS Q8
 * GEMM (or the f16 GEMM on expanded weights): the activations are copied
 * to f16 once, row-scaled (a_rows_f16), then the GEMM runs on f16 A.
 * When the weight is expanded for this call only, the copy and the
 * expansion are one launch (s3k_cast_rows_expand). */
static enum sam3_error q8_dl_cast(struct s3k_gemm *g, void *stream)
{
	struct s3k_gemm h = *g;
	if (q8_expands_per_call(&h) && h.batch == 1) {
		size_t a_bytes;
		const size_t abuf = a_rows_f16_bytes(&h, &a_bytes);
		const size_t wbytes = (size_t)h.N * h.K * 2;
		void *buf = NULL;
		enum sam3_error err = s3h_scratch_alloc(
			&buf, a_bytes + ((abuf - a_bytes + 255) & ~(size_t)255) + wbytes + (size_t)h.N * 4,
			stream);
		if (err != SAM3_OK)
			return err;
		float *rs = (float *)((char *)buf + a_bytes);
		uint16_t *w16 = (uint16_t *)((char *)buf + a_bytes +
					     ((abuf - a_bytes + 255) & ~(size_t)255));
		float *cs = (float *)((char *)w16 + wbytes);
		const int e = s3k_cast_rows_expand(h.a_kind, h.a, h.lda, buf, rs, h.M, h.K, h.b, w16, cs,
						   h.N, stream);
		if (e == (int)hipSuccess) {
			h.a = buf;
			h.a_kind = S3K_F16;
			h.lda = h.K;
			h.stride_a = 0;
			h.rs = rs;
			h.rs_sb = 0;
			h.flags |= S3K_EPI_ROWSCALE;
			h.b = w16;
			h.b_kind = S3K_F16;
			h.ldb = h.K;
			h.cs = cs;
			h.cs_sb = 0;
			h.flags |= S3K_EPI_COLSCALE;
			err = s3h_hip(s3k_gemm_launch_path(&h, S3K_PATH_MFMA, stream),
				      "matmul_q8 f16 gemm");
			enum sam3_error ferr = s3h_scratch_free(buf, stream);
			return err != SAM3_OK ? err : ferr;
		}
		(void)hipGetLastError();
		err = s3h_scratch_free(buf, stream);
		if (err != SAM3_OK)
			return err;
		if (e != (int)hipErrorInvalidValue)
			return s3h_hip(e, "matmul_q8 cast + expand");
	}
	void *tmp = NULL;
	enum sam3_error err = a_rows_f16(&h, &tmp, stream);
	if (err == SAM3_OK)
		err = q8_f16_gemm(&h, stream);
	if (tmp) {
		enum sam3_error ferr = s3h_scratch_free(tmp, stream);
		if (err == SAM3_OK)
			err = ferr;
	}
	return err;
}

static int q8_dl_wants_cast(const struct s3k_gemm *g)
{
	return g->b_kind == S3K_Q8 && g->a_kind != S3K_F16 && s3k_dlq8_eligible(g);
}

/* f32 x f32 with W [N,K] on the bf16 MFMA GEMM: A and W are split once
 * into bf16 hi/lo planes laid out along a tripled k, A' = [Ah | Al | Ah]
 * and W' = [Wh | Wh | Wl], so that one bf16 GEMM over 3K accumulates
 * Ah*Wh + Al*Wh + Ah*Wl in f32; the dropped Al*Wl term is below 2^-16 of
 * each product. */
static int f32_split_wanted(const struct s3k_gemm *g)
{
	if (!s3h_settings()->f32_split)
		return 0;
	return g->a_kind == S3K_F32 && g->b_kind == S3K_F32 && g->c_kind == S3K_F32 &&
	       (g->flags & S3K_B_NT) && g->batch == 1 && g->K % 8 == 0 && g->lda % 4 == 0 &&
	       g->ldb % 4 == 0 && !(((uintptr_t)g->a | (uintptr_t)g->b) & 15u) &&
	       (long long)g->M * 3 * g->K * 2 <= 0x7FFFFFF0LL &&
	       (long long)g->N * 3 * g->K * 2 <= 0x7FFFFFF0LL &&
	       (long long)g->M * g->N * g->K >= (1LL << 24);
}

/* a_planes: A already split by its producer ([M, 3K] = [hi|lo|hi]), or
 * NULL to split g->a here. */
static enum sam3_error f32_split_gemm(const struct s3k_gemm *g, const void *a_planes, void *stream)
{
	const size_t abytes = (size_t)g->M * 3 * g->K * 2, bbytes = (size_t)g->N * 3 * g->K * 2;
	void *a3 = NULL, *b3 = NULL;
	int own_b = 1;
	enum sam3_error err = SAM3_OK;
	if (!a_planes) {
		err = s3h_scratch_alloc(&a3, abytes, stream);
		if (err == SAM3_OK)
			err = s3h_hip(s3k_split3_bf16((const float *)g->a, a3, g->M, g->K, g->lda, 0, stream),
				      "matmul f32 split A");
	}
	if (err == SAM3_OK && g->ldb == g->K)
		err = prep_weight(g->b, (size_t)g->N * g->K * 4, S3H_PREP_SPLIT_W, g->N, g->K, g->K,
				  bbytes, S3K_F32, prep_split_w, stream, &b3, &own_b);
	else if (err == SAM3_OK) {
		err = s3h_scratch_alloc(&b3, bbytes, stream);
		if (err == SAM3_OK)
			err = s3h_hip(s3k_split3_bf16((const float *)g->b, b3, g->N, g->K, g->ldb, 1, stream),
				      "matmul f32 split W");
	}
	if (err == SAM3_OK) {
		struct s3k_gemm h = *g;
		h.a = a_planes ? a_planes : a3;
		h.b = b3;
		h.a_kind = h.b_kind = S3K_BF16;
		h.K = 3 * g->K;
		h.lda = h.ldb = 3 * g->K;
		err = s3h_hip(s3k_gemm_launch_path(&h, S3K_PATH_MFMA, stream), "matmul f32 split gemm");
	}
	enum sam3_error ferr = SAM3_OK;
	if (b3 && own_b)
		ferr = s3h_scratch_free(b3, stream);
	if (a3) {
		enum sam3_error e2 = s3h_scratch_free(a3, stream);
		if (ferr == SAM3_OK)
			ferr = e2;
	}
	return err != SAM3_OK ? err : ferr;
}

static int q8_needs_unpack(const struct s3k_gemm *g)
{
	if (g->b_kind != S3K_Q8)
		return 0;
	if ((g->flags & S3K_B_NT) && g->K % 32 == 0)
		return 0;
	/* large enough for a GEMM to pay for the unpack pass */
	return g->K % 8 == 0 && g->M >= 64 && (long long)g->M * g->N * g->K >= (1LL << 21);
}

static enum sam3_error matmul_impl(int path, int a_dt, const void *a, int b_dt, const void *b,
				   int c_dt, void *c, int M, int N, int K, const void *bias,
				   int flags, void *stream)
{
	enum sam3_error err;

	if (M < 0 || N < 0 || K < 0) {
		s3h_error("matmul: negative size M=%d N=%d K=%d", M, N, K);
		return SAM3_EINVAL;
	}
	if (M == 0 || N == 0)
		return SAM3_OK;
	if (!a || !b || !c || ((flags & SAM3_HIP_BIAS) && !bias)) {
		s3h_error("matmul: NULL pointer");
		return SAM3_EINVAL;
	}
	err = check_kinds(a_dt, b_dt, c_dt);
	if (err != SAM3_OK)
		return err;

	struct s3k_gemm g;
	fill_gemm(&g, a_dt, a, b_dt, b, c_dt, c, M, N, K, bias, flags);

	if (path == 0) {
		if (q8_needs_unpack(&g))
			return q8_unpacked(&g, stream);
		if (f32_split_wanted(&g))
			return f32_split_gemm(&g, NULL, stream);
		if (s3k_gemm_path(&g) == S3K_PATH_MFMA && q8_dl_wants_cast(&g))
			return q8_dl_cast(&g, stream);
		if (g.b_kind == S3K_Q8 && g.a_kind == S3K_F16 && s3k_gemm_path(&g) == S3K_PATH_MFMA)
			return q8_f16_gemm(&g, stream);
		const int p0 = s3k_gemm_path(&g);
		if (p0 == S3K_PATH_NONE) {
			s3h_error("matmul: no kernel for M=%d N=%d K=%d", M, N, K);
			return SAM3_EINVAL;
		}
		return launch_a_safe(&g, p0, "matmul", stream);
	}
	if (path < S3K_PATH_MFMA || path > S3K_PATH_GENERIC) {
		s3h_error("matmul: unknown path %d", path);
		return SAM3_EINVAL;
	}
	if (path == S3K_PATH_MFMA && q8_needs_unpack(&g))
		return q8_unpacked(&g, stream);
	if (path == S3K_PATH_MFMA && f32_split_wanted(&g))
		return f32_split_gemm(&g, NULL, stream);
	if (path == S3K_PATH_MFMA && q8_dl_wants_cast(&g))
		return q8_dl_cast(&g, stream);
	return launch_a_safe(&g, path, "matmul", stream);
}

/* f32 activations times Q8_0 weights on the skinny kernels, which would
 * first copy A to f16 rows (launch_a_safe): A given already as f16 (an
 * operand a producer wrote) is read as it is. Producers are not asked to
 * write this form (s3h_matmul_a_format): their range flag makes
 * graph_eval wait for the GPU at its end, which costs a skinny chain more
 * than the row copy it saves. */
/* g reads A as the LayerNorm input ln (S3K_A_LN). */
static void use_ln_input(struct s3k_gemm *g, const struct s3h_ln_in *ln)
{
	g->a = ln->x;
	g->a_kind = S3K_F32;
	g->lda = g->K;
	g->flags |= S3K_A_LN;
	g->ln_g = ln->gamma;
	g->ln_b = ln->beta;
}

/* g reads A as v of one-key attention heads (S3K_A_ATT1). */
static void use_att1_input(struct s3k_gemm *g, const struct s3h_att1_in *at)
{
	g->a = at->v;
	g->a_kind = S3K_F32;
	g->lda = g->K;
	g->flags |= S3K_A_ATT1;
	g->att_q = at->q;
	g->att_k = at->k;
	g->att_mask = at->mask;
	g->att_scale = at->scale;
	g->att_D = at->D;
}

/* The forms whose A is a node that did not run (S3H_A_LN, S3H_A_ATT1):
 * the skinny kernel computes it from that node's inputs as it reads. */
static int a_folded(int a_fmt)
{
	return a_fmt == S3H_A_LN || a_fmt == S3H_A_ATT1;
}

/* The device rows a GEMM with A in form a_fmt reads. */
static const void *a_rows(int a_fmt, const void *a)
{
	return a_fmt == S3H_A_LN     ? (const void *)((const struct s3h_ln_in *)a)->x
	       : a_fmt == S3H_A_ATT1 ? (const void *)((const struct s3h_att1_in *)a)->v
				     : a;
}

static void use_folded_input(struct s3k_gemm *g, int a_fmt, const void *a)
{
	if (a_fmt == S3H_A_LN)
		use_ln_input(g, (const struct s3h_ln_in *)a);
	else
		use_att1_input(g, (const struct s3h_att1_in *)a);
}

/* The skinny launch takes g with its A as a LayerNorm's input (or v of
 * one-key attention). */
static int skinny_takes_ln(const struct s3k_gemm *g)
{
	return g->b_kind == S3K_Q8 && g->batch == 1 && s3k_gemm_path(g) == S3K_PATH_SKINNY &&
	       s3k_skinny_ok(g);
}

int s3h_matmul_ln_ok(int b_dt, const void *b, int M, int N, int K, int flags,
		     const struct s3h_ln_in *ln)
{
	if (b_dt != SAM3_DTYPE_Q8_0 || !(flags & SAM3_HIP_B_NT) || !ln || !ln->x || !b || M <= 0 ||
	    N <= 0 || K <= 0 || !s3h_settings()->ln_gemv_fold)
		return 0;
	struct s3k_gemm g;
	fill_gemm(&g, SAM3_DTYPE_F32, ln->x, b_dt, b, SAM3_DTYPE_F32, (void *)ln->x, M, N, K, NULL,
		  flags);
	use_ln_input(&g, ln);
	return skinny_takes_ln(&g);
}

int s3h_matmul_att1_ok(int b_dt, const void *b, int M, int N, int K, int flags,
		       const struct s3h_att1_in *at)
{
	if (b_dt != SAM3_DTYPE_Q8_0 || !(flags & SAM3_HIP_B_NT) || !at || !at->q || !at->k ||
	    !at->v || !b || M != 1 || N <= 0 || K <= 0 || !s3h_settings()->att_gemv_fold)
		return 0;
	struct s3k_gemm g;
	fill_gemm(&g, SAM3_DTYPE_F32, at->v, b_dt, b, SAM3_DTYPE_F32, (void *)at->v, M, N, K, NULL,
		  flags);
	use_att1_input(&g, at);
	return skinny_takes_ln(&g);
}

static int skinny_takes_f16(const struct s3k_gemm *g)
{
	if (g->a_kind != S3K_F32 || g->b_kind != S3K_Q8 || g->batch != 1 ||
	    s3k_gemm_path(g) != S3K_PATH_SKINNY)
		return 0;
	struct s3k_gemm h = *g;
	h.a_kind = S3K_F16;
	return s3k_gemm_path(&h) == S3K_PATH_SKINNY && rounds_a_to_f16(g, S3K_PATH_SKINNY);
}

int s3h_matmul_a_format(int a_dt, const void *a, int b_dt, const void *b, int c_dt, int M, int N,
			int K, int flags)
{
	if (check_kinds(a_dt, b_dt, c_dt) != SAM3_OK || M <= 0 || N <= 0 || K <= 0 || !a || !b)
		return S3H_A_PLAIN;
	struct s3k_gemm g;
	fill_gemm(&g, a_dt, a, b_dt, b, c_dt, (void *)a, M, N, K, NULL, flags);
	if (q8_needs_unpack(&g))
		return S3H_A_PLAIN;
	if (f32_split_wanted(&g))
		return S3H_A_PLANES;
	if (g.a_kind == S3K_F32 && s3k_gemm_path(&g) == S3K_PATH_MFMA && q8_dl_wants_cast(&g))
		return S3H_A_F16;
	return S3H_A_PLAIN;
}

enum sam3_error s3h_matmul_fmt(int a_fmt, int a_dt, const void *a, int b_dt, const void *b,
			       int c_dt, void *c, int M, int N, int K, const void *bias, int flags,
			       void *stream)
{
	if (a_fmt == S3H_A_PLAIN)
		return matmul_impl(0, a_dt, a, b_dt, b, c_dt, c, M, N, K, bias, flags, stream);
	if (M <= 0 || N <= 0 || K <= 0 || !a || !b || !c || ((flags & SAM3_HIP_BIAS) && !bias)) {
		s3h_error("matmul: bad prepared-operand call M=%d N=%d K=%d", M, N, K);
		return SAM3_EINVAL;
	}
	struct s3k_gemm g;
	fill_gemm(&g, a_dt, a, b_dt, b, c_dt, c, M, N, K, bias, flags);
	if (a_fmt == S3H_A_PLANES) {
		if (!f32_split_wanted(&g)) {
			s3h_error("matmul: A given as bf16 planes but the split GEMM cannot run");
			return SAM3_EINVAL;
		}
		return f32_split_gemm(&g, a, stream);
	}
	if (a_folded(a_fmt)) {
		use_folded_input(&g, a_fmt, a);
		if (!skinny_takes_ln(&g)) {
			s3h_error("matmul: the folded input form %d cannot be read by this GEMM", a_fmt);
			return SAM3_EINVAL;
		}
		return s3h_hip(s3k_gemm_launch_path(&g, S3K_PATH_SKINNY, stream),
			       "matmul skinny (folded input)");
	}
	if (a_fmt == S3H_A_F16 && skinny_takes_f16(&g)) {
		g.a_kind = S3K_F16;
		return s3h_hip(s3k_gemm_launch_path(&g, S3K_PATH_SKINNY, stream), "matmul skinny");
	}
	if (a_fmt == S3H_A_F16 && g.a_kind == S3K_F32 && q8_dl_wants_cast(&g)) {
		g.a_kind = S3K_F16;
		return q8_f16_gemm(&g, stream);
	}
	s3h_error("matmul: operand format %d does not fit this GEMM", a_fmt);
	return SAM3_EINVAL;
}

/* Whether the GEMM that s3h_matmul_fmt runs for A in form a_fmt ends in
 * the direct-to-LDS GEMM, which can write its f32 result as the operand
 * form out_fmt (S3H_A_PLANES or S3H_A_F16) of a following GEMM, or as f32
 * (S3H_A_PLAIN) with a residual added. f32 weights reach it through the
 * split GEMM, Q8_0 weights through their f16 expansion (f16 A only). b
 * is the weight's device address; a is used for its alignment only. */
int s3h_matmul_out_ok(int a_fmt, int a_dt, const void *a, int b_dt, const void *b, int M, int N,
		      int K, int flags, int out_fmt)
{
	static const char al[16] __attribute__((aligned(16)));
	if ((out_fmt != S3H_A_PLAIN && out_fmt != S3H_A_PLANES && out_fmt != S3H_A_F16) || M <= 0 ||
	    N <= 0 || K <= 0 || (out_fmt != S3H_A_PLAIN && N % 8) || !a || !b ||
	    check_kinds(a_dt, b_dt, SAM3_DTYPE_F32) != SAM3_OK)
		return 0;
	struct s3k_gemm g;
	fill_gemm(&g, a_dt, a, b_dt, b, SAM3_DTYPE_F32, (void *)al, M, N, K, NULL, flags);
	struct s3k_gemm h = g;
	h.a = h.b = al;
	if (b_dt == SAM3_DTYPE_F32) {
		if ((a_fmt != S3H_A_PLANES && a_fmt != S3H_A_PLAIN) || !f32_split_wanted(&g))
			return 0;
		h.a_kind = h.b_kind = S3K_BF16;
		h.K = 3 * K;
		h.lda = h.ldb = 3 * K;
		return s3k_dl_eligible(&h);
	}
	if (b_dt != SAM3_DTYPE_Q8_0 || a_fmt != S3H_A_F16 || a_dt != SAM3_DTYPE_F32)
		return 0;
	if (s3k_gemm_path(&h) == S3K_PATH_SKINNY)
		return 0; /* few rows: the Q8_0 blocks streamed, not an f16 copy */
	/* the expansion q8_f16_gemm makes */
	const int mode = s3h_settings()->q8_expand;
	if (!(g.flags & S3K_B_NT) || K % 32 || mode == 0 ||
	    (mode != 1 && M < S3H_Q8_EXPAND_MIN_M &&
	     !s3h_prep_cacheable(b, (size_t)N * (K / 32) * 36)))
		return 0;
	h.a_kind = h.b_kind = S3K_F16;
	h.ldb = K;
	return s3k_dl_eligible(&h);
}

/* A skinny Q8_0 GEMM (f32 out, batch 1) that adds a residual in its
 * epilogue: A f16 written by its producer (S3H_A_F16), or f32 (copied to
 * f16 rows first). */
static int skinny_res_fits(int a_fmt, const struct s3k_gemm *g)
{
	if (g->b_kind != S3K_Q8 || g->c_kind != S3K_F32 || g->batch != 1 || g->ldc != g->N ||
	    g->a_kind != S3K_F32)
		return 0;
	if (a_fmt == S3H_A_F16)
		return skinny_takes_f16(g);
	return a_fmt == S3H_A_PLAIN && s3k_gemm_path(g) == S3K_PATH_SKINNY;
}

/* s3h_matmul_res_ok / s3h_matmul_qkv_ok for A read as a LayerNorm's
 * input (the streaming skinny kernel with S3K_A_LN) or as v of one-key
 * attention (the f32 GEMV with S3K_A_ATT1). */
static int ln_skinny_fits(int a_fmt, int a_dt, const void *a, int b_dt, const void *b, int M,
			  int N, int K, int flags)
{
	if (a_dt != SAM3_DTYPE_F32)
		return 0;
	return a_fmt == S3H_A_LN
		       ? s3h_matmul_ln_ok(b_dt, b, M, N, K, flags, (const struct s3h_ln_in *)a)
		       : s3h_matmul_att1_ok(b_dt, b, M, N, K, flags, (const struct s3h_att1_in *)a);
}

/* Whether s3h_matmul_fmt_to can add an f32 [M, N] residual to this GEMM's
 * f32 result in its epilogue (no row map). */
int s3h_matmul_res_ok(int a_fmt, int a_dt, const void *a, int b_dt, const void *b, int M, int N,
		      int K, int flags)
{
	if (a_folded(a_fmt))
		return ln_skinny_fits(a_fmt, a_dt, a, b_dt, b, M, N, K, flags);
	if (s3h_matmul_out_ok(a_fmt, a_dt, a, b_dt, b, M, N, K, flags, S3H_A_PLAIN))
		return 1;
	if (M <= 0 || N <= 0 || K <= 0 || !a || !b ||
	    check_kinds(a_dt, b_dt, SAM3_DTYPE_F32) != SAM3_OK)
		return 0;
	static const char al[16] __attribute__((aligned(16)));
	struct s3k_gemm g;
	fill_gemm(&g, a_dt, a, b_dt, b, SAM3_DTYPE_F32, (void *)al, M, N, K, NULL, flags);
	g.a = al;
	return skinny_res_fits(a_fmt, &g);
}

/* The GEMM of s3h_matmul_fmt with its f32 result written as out_fmt:
 * bf16 planes [M, 3N] = [hi|lo|hi] per row, or f16 [M, N], with the
 * bias and GELU applied in f32 first, the values split3 / the f16 cast
 * of the f32 output would give. */
enum sam3_error s3h_matmul_fmt_to(int a_fmt, int out_fmt, int a_dt, const void *a, int b_dt,
				  const void *b, void *c, int M, int N, int K, const void *bias,
				  const void *res, const int *row_map, int flags, unsigned *ovf,
				  unsigned ovf_tag, unsigned *rowf, void *stream)
{
	const int fits = out_fmt == S3H_A_PLAIN && !row_map
				 ? s3h_matmul_res_ok(a_fmt, a_dt, a, b_dt, b, M, N, K, flags)
				 : s3h_matmul_out_ok(a_fmt, a_dt, a, b_dt, b, M, N, K, flags, out_fmt);
	if (!c || ((flags & SAM3_HIP_BIAS) && !bias) || (res && ((uintptr_t)res & 3u)) || !fits) {
		s3h_error("matmul: cannot write form %d (M=%d N=%d K=%d)", out_fmt, M, N, K);
		return SAM3_EINVAL;
	}
	if (a_folded(a_fmt) && (out_fmt != S3H_A_PLAIN || row_map)) {
		s3h_error("matmul: a folded input GEMM writes f32 rows only");
		return SAM3_EINVAL;
	}
	struct s3k_gemm g;
	fill_gemm(&g, a_dt, a_rows(a_fmt, a), b_dt, b, SAM3_DTYPE_F32, c, M, N, K, bias, flags);
	g.c_kind = out_fmt == S3H_A_PLANES ? S3K_C_PLANES
		 : out_fmt == S3H_A_F16     ? S3K_C_F16OP
					    : S3K_F32;
	g.ldc = out_fmt == S3H_A_PLANES ? 3 * N : N;
	if (out_fmt == S3H_A_F16) {
		g.ovf = ovf;
		g.ovf_tag = ovf_tag;
		g.rowf = ovf ? rowf : NULL;
	}
	if (res) {
		g.res = res;
		g.flags |= S3K_EPI_RES;
	}
	if (row_map) {
		if (out_fmt != S3H_A_PLAIN || row_map[0] <= 0 || row_map[1] <= 0 || row_map[2] <= 0 ||
		    M % ((long long)row_map[0] * row_map[1] * row_map[2])) {
			s3h_error("matmul: bad output row map");
			return SAM3_EINVAL;
		}
		g.rm_g = row_map[0];
		g.rm_d1 = row_map[1];
		g.rm_d2 = row_map[2];
	}
	if (a_folded(a_fmt)) {
		use_folded_input(&g, a_fmt, a);
		return s3h_hip(s3k_gemm_launch_path(&g, S3K_PATH_SKINNY, stream),
			       "matmul skinny (folded input)");
	}
	if (b_dt == SAM3_DTYPE_F32)
		return f32_split_gemm(&g, a_fmt == S3H_A_PLANES ? a : NULL, stream);
	if (out_fmt == S3H_A_PLAIN && !row_map && skinny_res_fits(a_fmt, &g)) {
		if (a_fmt == S3H_A_F16) {
			g.a_kind = S3K_F16;
			return s3h_hip(s3k_gemm_launch_path(&g, S3K_PATH_SKINNY, stream),
				       "matmul skinny");
		}
		return launch_a_safe(&g, S3K_PATH_SKINNY, "matmul skinny", stream);
	}
	g.a_kind = S3K_F16;
	return q8_f16_gemm(&g, stream);
}

static void fill_qkv(struct s3k_gemm *g, const struct s3h_qkv *q)
{
	for (int y = 0; y < 3; y++)
		g->qkv_out[y] = q->out[y];
	g->qkv_cos = q->cos_t;
	g->qkv_sin = q->sin_t;
	g->qkv_S = q->S;
	g->qkv_H = q->H;
	g->qkv_D = q->D;
	g->qkv_rope = q->rope;
	g->flags |= S3K_EPI_QKV;
}

/* A Q8_0 GEMM on the streaming skinny kernel that takes the head-split
 * stores (no RoPE): f32 activations read as they are (the kernel scales
 * rows into the f16 range itself) or an f16 operand a producer wrote. */
static int qkv_skinny(int a_fmt, int a_dt, const void *a, int b_dt, const void *b, int M, int N,
		      int K, int flags)
{
	if (b_dt != SAM3_DTYPE_Q8_0 || a_dt != SAM3_DTYPE_F32 || !(flags & SAM3_HIP_B_NT) ||
	    a_fmt == S3H_A_ATT1)
		return 0;
	if (a_fmt == S3H_A_LN)
		return ln_skinny_fits(a_fmt, a_dt, a, b_dt, b, M, N, K, flags);
	static const char al[16] __attribute__((aligned(16)));
	struct s3k_gemm g;
	fill_gemm(&g, a_dt, a, b_dt, b, SAM3_DTYPE_F32, (void *)al, M, N, K, NULL, flags);
	if (a_fmt == S3H_A_F16)
		return skinny_takes_f16(&g);
	return a_fmt == S3H_A_PLAIN && s3k_gemm_path(&g) == S3K_PATH_SKINNY &&
	       !rounds_a_to_f16(&g, S3K_PATH_SKINNY);
}

/* The kernel's conditions (s3k_gemm_launch_path) on the GEMM that
 * s3h_matmul_fmt_to would run, here for the operand geometry; the GEMM
 * itself must reach the direct-to-LDS kernel (s3h_matmul_out_ok) or,
 * without RoPE, the streaming skinny kernel. */
int s3h_matmul_qkv_ok(int a_fmt, int a_dt, const void *a, int b_dt, const void *b, int M, int N,
		      int K, int flags, const struct s3h_qkv *q)
{
	if (!q || (flags & SAM3_HIP_GELU) || q->D < 4 || (q->D & (q->D - 1)) || q->H <= 0 ||
	    q->S < 1 || M % q->S || (long long)q->H * q->D > (1 << 28) ||
	    (long long)q->S * q->D > 0x7FFFFFFFLL || N % (q->H * q->D))
		return 0;
	const int n_out = N / (q->H * q->D);
	if (n_out < 1 || n_out > 3 || q->rope < 0 || (q->rope >> n_out) ||
	    (q->rope && (!q->cos_t || !q->sin_t ||
			 (((uintptr_t)q->cos_t | (uintptr_t)q->sin_t) & 7u))))
		return 0;
	for (int y = 0; y < n_out; y++)
		if (!q->out[y] || ((uintptr_t)q->out[y] & 15u))
			return 0;
	if (!q->rope && qkv_skinny(a_fmt, a_dt, a, b_dt, b, M, N, K, flags))
		return 1;
	return !a_folded(a_fmt) && K % 64 == 0 && q->S >= 32 &&
	       s3h_matmul_out_ok(a_fmt, a_dt, a, b_dt, b, M, N, K, flags, S3H_A_PLAIN);
}

enum sam3_error s3h_matmul_qkv(int a_fmt, int a_dt, const void *a, int b_dt, const void *b, int M,
			       int N, int K, const void *bias, int flags, const struct s3h_qkv *q,
			       void *stream)
{
	if (((flags & SAM3_HIP_BIAS) && (!bias || ((uintptr_t)bias & 15u))) ||
	    !s3h_matmul_qkv_ok(a_fmt, a_dt, a, b_dt, b, M, N, K, flags, q)) {
		s3h_error("matmul: cannot store the attention operands (M=%d N=%d K=%d)", M, N, K);
		return SAM3_EINVAL;
	}
	struct s3k_gemm g;
	fill_gemm(&g, a_dt, a_fmt == S3H_A_LN ? ((const struct s3h_ln_in *)a)->x : a, b_dt, b,
		  SAM3_DTYPE_F32, q->out[0], M, N, K, bias, flags);
	fill_qkv(&g, q);
	if (!q->rope && qkv_skinny(a_fmt, a_dt, a, b_dt, b, M, N, K, flags)) {
		if (a_fmt == S3H_A_F16)
			g.a_kind = S3K_F16;
		if (a_fmt == S3H_A_LN)
			use_ln_input(&g, (const struct s3h_ln_in *)a);
		return s3h_hip(s3k_gemm_launch_path(&g, S3K_PATH_SKINNY, stream),
			       "matmul skinny (attention operands)");
	}
	if (b_dt == SAM3_DTYPE_F32)
		return f32_split_gemm(&g, a_fmt == S3H_A_PLANES ? a : NULL, stream);
	g.a_kind = S3K_F16;
	return q8_f16_gemm(&g, stream);
}

enum sam3_error sam3_hip_matmul(int a_dtype, const void *a, int b_dtype, const void *b,
				int c_dtype, void *c, int M, int N, int K,
				const void *bias, int flags, void *stream)
{
	return matmul_impl(0, a_dtype, a, b_dtype, b, c_dtype, c, M, N, K, bias, flags, stream);
}

enum sam3_error sam3_hip_matmul_on_path(int path, int a_dtype, const void *a,
					int b_dtype, const void *b, int c_dtype, void *c,
					int M, int N, int K, const void *bias, int flags,
					void *stream)
{
	return matmul_impl(path, a_dtype, a, b_dtype, b, c_dtype, c, M, N, K, bias, flags, stream);
}

int sam3_hip_matmul_path(int a_dtype, int b_dtype, int c_dtype, int M, int N, int K, int flags)
{
	static const char dummy[64] __attribute__((aligned(64)));
	if (check_kinds(a_dtype, b_dtype, c_dtype) != SAM3_OK || M <= 0 || N <= 0 || K < 0)
		return S3K_PATH_NONE;
	struct s3k_gemm g;
	fill_gemm(&g, a_dtype, dummy, b_dtype, dummy, c_dtype, (void *)dummy, M, N, K,
		  dummy, flags);
	if (q8_needs_unpack(&g))
		return S3K_PATH_MFMA;
	return s3k_gemm_path(&g);
}

enum sam3_error sam3_hip_matmul_batched(int dtype, const void *a, const void *b, void *c,
					int batch, int M, int N, int K,
					long long stride_a, long long stride_b,
					long long stride_c, int flags, void *stream)
{
	if (batch < 0 || M < 0 || N < 0 || K < 0) {
		s3h_error("matmul_batched: negative size");
		return SAM3_EINVAL;
	}
	if (batch == 0 || M == 0 || N == 0)
		return SAM3_OK;
	if (!a || !b || !c) {
		s3h_error("matmul_batched: NULL pointer");
		return SAM3_EINVAL;
	}
	if (!is_float_dtype(dtype)) {
		s3h_error("matmul_batched: unsupported dtype %d", dtype);
		return SAM3_EDTYPE;
	}
	if (flags & SAM3_HIP_BIAS) {
		s3h_error("matmul_batched: bias is not supported on batches");
		return SAM3_EINVAL;
	}
	struct s3k_gemm g;
	fill_gemm(&g, dtype, a, dtype, b, dtype, c, M, N, K, NULL, flags);
	g.batch = batch;
	g.stride_a = stride_a;
	g.stride_b = stride_b;
	g.stride_c = stride_c;
	return s3h_hip(s3k_gemm_launch(&g, stream), "matmul_batched");
}

/* Activation rows from which a batched stream of Q8 weights with shared
 * activations runs on the tiled Q8 GEMM (one tile of all rows per weight
 * tile, full k per workgroup) instead of the skinny kernel (k split over
 * a workgroup's waves); K <= 256 takes the GEMM at any M (the skinny
 * kernel's k split leaves half its waves idle there). Measured on every
 * config-4 shape. SAM3_HIP_Q8_BATCH_PATH=1 forces the skinny kernel, =2
 * the GEMM. */
#define S3H_Q8_BATCH_GEMM_M 8

enum sam3_error sam3_hip_matmul_q8_batched(int a_dtype, const void *a, const void *w,
					   void *c, int batch, int M, int N, int K,
					   long long stride_a, long long stride_w,
					   long long stride_c, const void *bias, int flags,
					   void *stream)
{
	if (batch < 0 || M < 0 || N < 0 || K < 0 || stride_a < 0 || stride_w < 0 || stride_c < 0) {
		s3h_error("matmul_q8_batched: negative size or stride");
		return SAM3_EINVAL;
	}
	if (batch == 0 || M == 0 || N == 0)
		return SAM3_OK;
	if (!a || !w || !c || ((flags & SAM3_HIP_BIAS) && !bias)) {
		s3h_error("matmul_q8_batched: NULL pointer");
		return SAM3_EINVAL;
	}
	if (!is_float_dtype(a_dtype)) {
		s3h_error("matmul_q8_batched: unsupported activation dtype %d", a_dtype);
		return SAM3_EDTYPE;
	}
	if (K % 32) {
		s3h_error("matmul_q8_batched: K=%d is not a multiple of 32", K);
		return SAM3_EINVAL;
	}
	flags = (flags & (SAM3_HIP_BIAS | SAM3_HIP_GELU)) | SAM3_HIP_B_NT;
	struct s3k_gemm g;
	fill_gemm(&g, a_dtype, a, SAM3_DTYPE_Q8_0, w, SAM3_DTYPE_F32, c, M, N, K, bias, flags);
	g.batch = batch;
	g.stride_a = stride_a;
	g.stride_b = stride_w;
	g.stride_c = stride_c;
	/* one f32 activation row: the f32 GEMV reads it as it is (a stream of
	 * K = 256 weights only on the persistent q8_gemv_tasks, 4.35 TB/s;
	 * one workgroup per task would give 3.2, the tiled GEMM below 3.7) */
	if (a_dtype == SAM3_DTYPE_F32 && M == 1 && K % 256 == 0 &&
	    (K > 256 || batch == 1 || s3k_gemv_tasks_take(&g)) &&
	    s3h_settings()->gemv_f32 &&
	    s3h_settings()->q8_batch_path != 2 && s3k_gemm_path(&g) == S3K_PATH_SKINNY)
		return s3h_hip(s3k_gemm_launch(&g, stream), "matmul_q8_batched gemv");
	if (s3k_gemm_path(&g) == S3K_PATH_SKINNY) {
		/* f32/bf16 activations are copied to f16 once, row-scaled
		 * (a_rows_f16; slices sharing them, at stride 0, share the copy),
		 * so each workgroup moves half the activation bytes */
		struct s3k_gemm h = g;
		void *a16 = NULL;
		enum sam3_error err = SAM3_OK;
		if (a_dtype != SAM3_DTYPE_F16)
			err = a_rows_f16(&h, &a16, stream);
		if (err == SAM3_OK) {
			const int force = s3h_settings()->q8_batch_path;
			/* 2-16 rows over enough weight tasks: the persistent
			 * q8_stream_tasks (skinny launch) before the GEMM */
			const int tasks = force != 2 && s3k_stream_tasks_take(&h);
			const int gemm = h.a_kind == S3K_F16 && batch > 1 && !tasks &&
					 (force == 2 ||
					  (force != 1 && (M >= S3H_Q8_BATCH_GEMM_M || K <= 256))) &&
					 s3k_dlq8_eligible(&h);
			/* the GEMM with the weight-row factors of every slice */
			err = gemm ? launch_a_safe(&h, S3K_PATH_MFMA, "matmul_q8_batched gemm", stream)
				   : s3h_hip(s3k_gemm_launch(&h, stream), "matmul_q8_batched");
		}
		if (a16) {
			enum sam3_error ferr = s3h_scratch_free(a16, stream);
			if (err == SAM3_OK)
				err = ferr;
		}
		return err;
	}
	/* one launch per slice on the kernel sam3_hip_matmul picks */
	const size_t es = s3h_dtype_size(a_dtype);
	for (int s = 0; s < batch; ++s) {
		enum sam3_error err = matmul_impl(
			0, a_dtype, (const char *)a + (size_t)s * stride_a * es, SAM3_DTYPE_Q8_0,
			(const char *)w + (size_t)s * stride_w, SAM3_DTYPE_F32,
			(float *)c + (size_t)s * stride_c, M, N, K, bias, flags, stream);
		if (err != SAM3_OK)
			return err;
	}
	return SAM3_OK;
}

/* sam3_hip_matmul for Q8_0 weights [N,K] without any allocation: the
 * row-scaled f16 copy of the activations that the MFMA and GEMV kernels
 * read, and the weight-row factors of the MFMA kernels, go to the
 * library's fixed per-device scratch array (s3k_noalloc_scratch), and
 * the Q8_0 weights are read in place (never expanded). With the
 * expansion off (SAM3_HIP_Q8_EXPAND=0) sam3_hip_matmul runs the same
 * kernels on the same values, so the results have the same bits; at the
 * default setting sam3_hip_matmul expands large weights to f16 (one
 * rounding of q*scale instead of the scale's and the product's) and the
 * two agree within the f32 tolerance. Calls that overlap on one device
 * (two threads, or two streams) share the array and race. */
enum sam3_error sam3_hip_matmul_q8_noalloc(int a_dtype, const void *a, const void *w, void *c,
					   int M, int N, int K, const void *bias, int flags,
					   void *stream)
{
	if (M < 0 || N < 0 || K < 0) {
		s3h_error("matmul_q8_noalloc: negative size M=%d N=%d K=%d", M, N, K);
		return SAM3_EINVAL;
	}
	if (M == 0 || N == 0)
		return SAM3_OK;
	if (!a || !w || !c || ((flags & SAM3_HIP_BIAS) && !bias)) {
		s3h_error("matmul_q8_noalloc: NULL pointer");
		return SAM3_EINVAL;
	}
	if (!is_float_dtype(a_dtype)) {
		s3h_error("matmul_q8_noalloc: unsupported activation dtype %d", a_dtype);
		return SAM3_EDTYPE;
	}
	if (K % 32) {
		s3h_error("matmul_q8_noalloc: K=%d is not a multiple of 32 (W must be whole Q8_0 "
			  "blocks per row)", K);
		return SAM3_EINVAL;
	}
	flags = (flags & (SAM3_HIP_BIAS | SAM3_HIP_GELU)) | SAM3_HIP_B_NT;
	struct s3k_gemm g;
	fill_gemm(&g, a_dtype, a, SAM3_DTYPE_Q8_0, w, SAM3_DTYPE_F32, c, M, N, K, bias, flags);
	const int path = s3k_gemm_path(&g);
	if (path == S3K_PATH_NONE) {
		s3h_error("matmul_q8_noalloc: no kernel for M=%d N=%d K=%d", M, N, K);
		return SAM3_EINVAL;
	}
	const int cast = rounds_a_to_f16(&g, path), fac = path == S3K_PATH_MFMA;
	if (!cast && !fac)
		return s3h_hip(s3k_gemm_launch_path(&g, path, stream), "matmul_q8_noalloc");
	/* [f16 activations, row factors | weight-row factors] */
	size_t a_bytes = 0, cap = 0;
	const size_t abuf = cast ? (a_rows_f16_bytes(&g, &a_bytes) + 255) & ~(size_t)255 : 0;
	const size_t need = abuf + (fac ? (size_t)N * 4 : 0);
	void *buf = NULL;
	enum sam3_error err = s3h_hip(s3k_noalloc_scratch(&buf, &cap), "matmul_q8_noalloc: scratch");
	if (err != SAM3_OK)
		return err;
	if (need > cap) {
		s3h_error("matmul_q8_noalloc: M=%d N=%d K=%d needs %zu bytes of scratch for the f16 "
			  "activations and weight factors, more than the %zu the library holds per "
			  "device", M, N, K, need, cap);
		return SAM3_EINVAL;
	}
	struct s3k_gemm h = g;
	if (cast) {
		err = a_rows_f16_into(&h, buf, stream);
		if (err != SAM3_OK)
			return err;
	}
	if (fac && q8_wauto_ok(&g)) {
		h.flags |= S3K_Q8_WAUTO; /* the kernel finds the weight-row factors */
	} else if (fac) {
		float *cs = (float *)((char *)buf + abuf);
		err = s3h_hip(s3k_q8_wfactors(w, cs, K, N, 1, 1, 0, stream),
			      "matmul_q8_noalloc weight factors");
		if (err != SAM3_OK)
			return err;
		h.cs = cs;
		h.cs_sb = 0;
		h.flags |= S3K_EPI_COLSCALE;
	}
	return s3h_hip(s3k_gemm_launch_path(&h, path, stream), "matmul_q8_noalloc");
}

/* ------------------------------------------------------------------ */
/* Attention                                                            */
/* ------------------------------------------------------------------ */
enum sam3_error sam3_hip_sdpa_on_path(int path, int dtype, const void *q, const void *k,
				      const void *v, const float *mask, void *out, int BH,
				      int Sq, int Sk, int D, void *stream)
{
	if (BH < 0 || Sq < 0 || Sk < 0 || D <= 0) {
		s3h_error("sdpa: negative size or head_dim <= 0");
		return SAM3_EINVAL;
	}
	if (!is_float_dtype(dtype)) {
		s3h_error("sdpa: dtype %d is not F32, F16 or BF16", dtype);
		return SAM3_EDTYPE;
	}
	if ((long long)BH * Sq == 0)
		return SAM3_OK;
	if (!q || !out || (Sk > 0 && (!k || !v))) {
		s3h_error("sdpa: NULL tensor");
		return SAM3_EINVAL;
	}
	if ((uintptr_t)mask & 3u) {
		s3h_error("sdpa: mask must be 4-byte aligned");
		return SAM3_EINVAL;
	}
	const int best = s3k_attn_path(dtype, q, k, v, out, BH, Sq, Sk, D);
	if (!best) {
		s3h_error("sdpa: no kernel for D=%d (D <= 512, element-aligned tensors)", D);
		return SAM3_EINVAL;
	}
	if (path != 0 && path != S3K_ATTN_GENERIC && path != S3K_ATTN_SMALL &&
	    !(path == S3K_ATTN_MFMA && best == path)) {
		s3h_error("sdpa: kernel %d cannot run this problem", path);
		return SAM3_EINVAL;
	}
	return s3h_hip(s3k_attn(path, dtype, q, k, v, mask, out, BH, Sq, Sk, D, stream), "sdpa");
}

enum sam3_error sam3_hip_sdpa(int dtype, const void *q, const void *k, const void *v,
			      const float *mask, void *out, int BH, int Sq, int Sk, int D,
			      void *stream)
{
	return sam3_hip_sdpa_on_path(0, dtype, q, k, v, mask, out, BH, Sq, Sk, D, stream);
}

/* ------------------------------------------------------------------ */
/* Q8_0 format on the device                                            */
/* ------------------------------------------------------------------ */
enum sam3_error sam3_hip_q8_quantize(const float *src, void *dst_blocks, int nelems,
				     void *stream)
{
	if (nelems < 0 || (nelems > 0 && (!src || !dst_blocks))) {
		s3h_error("q8_quantize: NULL pointer or negative size");
		return SAM3_EINVAL;
	}
	if (((uintptr_t)src & 3u) || ((uintptr_t)dst_blocks & 3u)) {
		s3h_error("q8_quantize: pointers must be 4-byte aligned");
		return SAM3_EINVAL;
	}
	return s3h_hip(s3k_q8_quantize(src, dst_blocks, nelems, stream), "q8_quantize");
}

enum sam3_error sam3_hip_q8_dequantize(const void *src_blocks, float *dst, int nelems,
				       void *stream)
{
	if (nelems < 0 || (nelems > 0 && (!src_blocks || !dst))) {
		s3h_error("q8_dequantize: NULL pointer or negative size");
		return SAM3_EINVAL;
	}
	if (((uintptr_t)src_blocks & 3u) || ((uintptr_t)dst & 3u)) {
		s3h_error("q8_dequantize: pointers must be 4-byte aligned");
		return SAM3_EINVAL;
	}
	return s3h_hip(s3k_q8_dequantize(src_blocks, dst, nelems, stream), "q8_dequantize");
}

/* ------------------------------------------------------------------ */
/* Node-level kernels                                                   */
/* ------------------------------------------------------------------ */

/* Shapes as the reference reads them: M = dims[n-2] (1 for 1-D), K =
 * dims[n-1]; B: K = dims[n-2], N = dims[n-1] (cpu_matmul_q8.c:187-213). */
static enum sam3_error node_shape(const struct sam3_node *node, const char *who,
				  int a_dt, int b_dt, int *M, int *N, int *K)
{
	if (!node || node->n_inputs < 2 || !node->inputs[0] || !node->inputs[1] ||
	    !node->output) {
		s3h_error("%s: NULL tensor", who);
		return SAM3_EINVAL;
	}
	const struct sam3_tensor *a = node->inputs[0], *b = node->inputs[1];
	const struct sam3_tensor *c = node->output;
	if ((int)a->dtype != a_dt || (int)b->dtype != b_dt) {
		s3h_error("%s: unsupported dtype (a=%d b=%d)", who, a->dtype, b->dtype);
		return SAM3_EINVAL;
	}
	if (b_dt == SAM3_DTYPE_Q8_0 && c->dtype != SAM3_DTYPE_F32) {
		s3h_error("%s: expected F32 x Q8_0 -> F32", who);
		return SAM3_EINVAL;
	}
	if (a->n_dims < 1 || b->n_dims < 1) {
		s3h_error("%s: need at least 1D tensors", who);
		return SAM3_EINVAL;
	}
	int ka, kb;
	if (a->n_dims == 1) {
		*M = 1;
		ka = a->dims[0];
	} else {
		*M = a->dims[a->n_dims - 2];
		ka = a->dims[a->n_dims - 1];
	}
	if (b->n_dims == 1) {
		kb = b->dims[0];
		*N = 1;
	} else {
		kb = b->dims[b->n_dims - 2];
		*N = b->dims[b->n_dims - 1];
	}
	if (ka != kb) {
		s3h_error("%s: K mismatch %d != %d", who, ka, kb);
		return SAM3_EINVAL;
	}
	*K = ka;
	if (s3h_nelems(c) != (long long)(*M) * (*N)) {
		s3h_error("%s: output size mismatch %lld != %lld", who, s3h_nelems(c),
			  (long long)(*M) * (*N));
		return SAM3_EINVAL;
	}
	return SAM3_OK;
}

static enum sam3_error node_matmul(const struct sam3_node *node, const char *who, int dt_a,
				   int dt_b, int dt_c, void *stream)
{
	int M, N, K;
	enum sam3_error err = node_shape(node, who, dt_a, dt_b, &M, &N, &K);
	if (err != SAM3_OK)
		return err;
	return sam3_hip_matmul(dt_a, node->inputs[0]->data, dt_b, node->inputs[1]->data, dt_c,
			       node->output->data, M, N, K, NULL, 0, stream);
}

enum sam3_error sam3_hip_kernel_matmul(const struct sam3_node *node, void *stream)
{
	return node_matmul(node, "matmul", SAM3_DTYPE_F32, SAM3_DTYPE_F32, SAM3_DTYPE_F32, stream);
}

enum sam3_error sam3_hip_kernel_matmul_f16(const struct sam3_node *node, void *stream)
{
	return node_matmul(node, "matmul_f16", SAM3_DTYPE_F16, SAM3_DTYPE_F16, SAM3_DTYPE_F16,
			   stream);
}

enum sam3_error sam3_hip_kernel_matmul_bf16(const struct sam3_node *node, void *stream)
{
	return node_matmul(node, "matmul_bf16", SAM3_DTYPE_BF16, SAM3_DTYPE_BF16,
			   SAM3_DTYPE_BF16, stream);
}

enum sam3_error sam3_hip_kernel_matmul_q8(const struct sam3_node *node, void *stream)
{
	return node_matmul(node, "matmul_q8", SAM3_DTYPE_F32, SAM3_DTYPE_Q8_0, SAM3_DTYPE_F32,
			   stream);
}

/* ADD: same shape, or y broadcast over the last dim of x (a bias). */
enum sam3_error s3h_add(const struct sam3_node *node, void *stream)
{
	if (node->n_inputs < 2 || !node->inputs[0] || !node->inputs[1] || !node->output) {
		s3h_error("add: NULL tensor");
		return SAM3_EINVAL;
	}
	const struct sam3_tensor *x = node->inputs[0], *y = node->inputs[1];
	const long long nx = s3h_nelems(x), ny = s3h_nelems(y);
	const int last = x->n_dims >= 1 ? x->dims[x->n_dims - 1] : 1;
	if (s3h_nelems(node->output) != nx) {
		s3h_error("add: output size mismatch");
		return SAM3_EINVAL;
	}
	if (ny == nx)
		return s3h_hip(s3k_add_same(x->dtype, x->data, y->data, node->output->data, nx,
					    stream), "add");
	if (ny == last && last > 0)
		return s3h_hip(s3k_bias_add(x->dtype, x->data, y->data, node->output->data,
					    nx / last, last, stream), "add");
	s3h_error("add: broadcast of %lld over %lld elements is not supported", ny, nx);
	return SAM3_EINVAL;
}

enum sam3_error s3h_gelu(const struct sam3_node *node, void *stream)
{
	if (node->n_inputs < 1 || !node->inputs[0] || !node->output) {
		s3h_error("gelu: NULL tensor");
		return SAM3_EINVAL;
	}
	const long long n = s3h_nelems(node->inputs[0]);
	if (s3h_nelems(node->output) != n) {
		s3h_error("gelu: output size mismatch");
		return SAM3_EINVAL;
	}
	return s3h_hip(s3k_gelu(node->inputs[0]->dtype, node->inputs[0]->data,
				node->output->data, n, stream), "gelu");
}

/* CAST (cpu_kernel_cast, cpu_cast.c:162-215): params[0] is the target
 * dtype and must be the output's; the same dtype is a copy; f32, f16 and
 * bf16 convert into each other. hw 0 converts bit-exactly as half.h
 * does; hw 1 with the hardware conversion instructions. */
int s3h_cast_ok(const struct sam3_node *node)
{
	if (node->n_inputs < 1 || !node->inputs[0] || !node->output)
		return 0;
	const int src = node->inputs[0]->dtype, dst = node->params[0];
	return dst == (int)node->output->dtype && is_float_dtype(src) && is_float_dtype(dst) &&
	       s3h_nelems(node->output) == s3h_nelems(node->inputs[0]);
}

static enum sam3_error cast_run(const struct sam3_node *node, int hw, void *stream)
{
	if (!node || node->n_inputs < 1 || !node->inputs[0] || !node->output) {
		s3h_error("cast: NULL tensor");
		return SAM3_EINVAL;
	}
	const int src = node->inputs[0]->dtype, dst = node->params[0];
	if (dst != (int)node->output->dtype) {
		s3h_error("cast: output dtype %d != params[0] %d", node->output->dtype, dst);
		return SAM3_EINVAL;
	}
	const long long n = s3h_nelems(node->inputs[0]);
	if (s3h_nelems(node->output) != n) {
		s3h_error("cast: output has %lld elements, input %lld", s3h_nelems(node->output), n);
		return SAM3_EINVAL;
	}
	if (n > 0 && (!node->inputs[0]->data || !node->output->data)) {
		s3h_error("cast: tensor without data");
		return SAM3_EINVAL;
	}
	if (src == dst)
		return n > 0 ? s3h_hip(hipMemcpyAsync(node->output->data, node->inputs[0]->data,
						      (size_t)n * s3h_dtype_size(src),
						      hipMemcpyDeviceToDevice, (hipStream_t)stream),
				       "cast (copy)")
			     : SAM3_OK;
	if (!is_float_dtype(src) || !is_float_dtype(dst)) {
		s3h_error("cast: unsupported %d -> %d", src, dst);
		return SAM3_EDTYPE;
	}
	return s3h_hip(s3k_cast(src, dst, node->inputs[0]->data, node->output->data, n, hw, stream),
		       "cast");
}

enum sam3_error sam3_hip_kernel_cast(const struct sam3_node *node, void *stream)
{
	return cast_run(node, 0, stream);
}

enum sam3_error sam3_hip_cast_on_path(int path, const struct sam3_node *node, void *stream)
{
	if (path != 1 && path != 2) {
		s3h_error("cast: unknown path %d", path);
		return SAM3_EINVAL;
	}
	return cast_run(node, path == 2, stream);
}

/* TRANSPOSE of the last two dims (params all zero, or the permutation
 * that swaps the last two axes; cpu_transpose.c:330-348). Other
 * permutations are not run here. */
int s3h_transpose_is_swap(const struct sam3_node *node)
{
	const struct sam3_tensor *in = node->inputs[0];
	const int nd = in->n_dims;
	if (nd < 2 || nd > SAM3_MAX_DIMS)
		return 0;
	int zero = 1;
	for (int i = 0; i < nd; i++)
		if (node->params[i] != 0)
			zero = 0;
	if (zero)
		return 1;
	for (int i = 0; i < nd - 2; i++)
		if (node->params[i] != i)
			return 0;
	return node->params[nd - 2] == nd - 1 && node->params[nd - 1] == nd - 2;
}

/* Axes of a TRANSPOSE node as cpu_kernel_transpose reads them
 * (cpu_transpose.c:330-348): params[0..nd-1]; all zero means the legacy
 * swap of the last two dims. */
static void transpose_axes(const struct sam3_node *node, int nd, int *axes)
{
	int any = 0;
	for (int i = 0; i < nd; i++) {
		axes[i] = node->params[i];
		if (axes[i])
			any = 1;
	}
	if (!any) {
		for (int i = 0; i < nd; i++)
			axes[i] = i;
		if (nd >= 2) {
			axes[nd - 2] = nd - 1;
			axes[nd - 1] = nd - 2;
		}
	}
}

int s3h_transpose_ok(const struct sam3_node *node)
{
	if (node->n_inputs < 1 || !node->inputs[0] || !node->output)
		return 0;
	const struct sam3_tensor *in = node->inputs[0];
	const int nd = in->n_dims;
	if (nd < 1 || nd > 4 || s3h_dtype_size(in->dtype) == 0 ||
	    s3h_nelems(node->output) != s3h_nelems(in))
		return 0;
	int axes[4], seen = 0;
	transpose_axes(node, nd, axes);
	for (int i = 0; i < nd; i++) {
		if (axes[i] < 0 || axes[i] >= nd || ((seen >> axes[i]) & 1))
			return 0;
		seen |= 1 << axes[i];
	}
	return 1;
}

enum sam3_error s3h_transpose(const struct sam3_node *node, void *stream)
{
	if (node->n_inputs < 1 || !node->inputs[0] || !node->output) {
		s3h_error("transpose: NULL tensor");
		return SAM3_EINVAL;
	}
	const struct sam3_tensor *in = node->inputs[0];
	if (s3h_dtype_size(in->dtype) == 0) {
		s3h_error("transpose: dtype %d has no element size", in->dtype);
		return SAM3_EDTYPE;
	}
	if (!s3h_transpose_ok(node)) {
		s3h_error("transpose: need 1-4 dims, a permutation in params and a same-size output");
		return SAM3_EINVAL;
	}
	const int nd = in->n_dims;
	if (nd >= 2 && s3h_transpose_is_swap(node)) {
		const int rows = in->dims[nd - 2], cols = in->dims[nd - 1];
		const long long batch = rows && cols ? s3h_nelems(in) / ((long long)rows * cols) : 0;
		return s3h_hip(s3k_transpose2d((int)s3h_dtype_size(in->dtype), in->data,
					       node->output->data, (int)batch, rows, cols, stream),
			       "transpose");
	}
	int axes[4];
	transpose_axes(node, nd, axes);
	return s3h_hip(s3k_permute((int)s3h_dtype_size(in->dtype), in->data, node->output->data,
				   nd, in->dims, axes, stream),
		       "transpose");
}

/* An f32 TRANSPOSE that keeps its last axis, with its output read as rows
 * of K values by a GEMM that converts A first: written in that operand
 * form (S3H_A_PLANES or S3H_A_F16) by s3h_transpose_to. */
int s3h_transpose_to_ok(const struct sam3_node *node, int K)
{
	if (!s3h_transpose_ok(node) || node->inputs[0]->dtype != SAM3_DTYPE_F32 || K <= 0 || K % 4)
		return 0;
	const struct sam3_tensor *in = node->inputs[0];
	const int nd = in->n_dims;
	int axes[4];
	transpose_axes(node, nd, axes);
	return axes[nd - 1] == nd - 1 && in->dims[nd - 1] % 4 == 0 && s3h_nelems(in) % K == 0;
}

enum sam3_error s3h_transpose_to(const struct sam3_node *node, const void *src, void *dst, int fmt,
				 int K, unsigned *ovf, unsigned ovf_tag, void *stream)
{
	if (!s3h_transpose_to_ok(node, K) || (fmt != S3H_A_PLANES && fmt != S3H_A_F16)) {
		s3h_error("transpose: cannot write GEMM operand form %d (K=%d)", fmt, K);
		return SAM3_EINVAL;
	}
	const struct sam3_tensor *in = node->inputs[0];
	int axes[4];
	transpose_axes(node, in->n_dims, axes);
	return s3h_hip(s3k_permute_to(fmt == S3H_A_PLANES ? S3K_LN_PLANES : S3K_LN_F16,
				      (const float *)src, dst, in->n_dims, in->dims, axes, K, ovf, ovf_tag,
				      stream),
		       "transpose (GEMM operand)");
}

/* LAYERNORM (cpu_layernorm.c:198-254 and its bf16/f16 twins): the last
 * dim is normalized; gamma and beta (optional) have the input's dtype. */
int s3h_layernorm_ok(const struct sam3_node *node)
{
	if (node->n_inputs < 1 || !node->inputs[0] || !node->output)
		return 0;
	const struct sam3_tensor *in = node->inputs[0];
	if (!is_float_dtype(in->dtype) || in->n_dims < 1 || node->output->dtype != in->dtype ||
	    s3h_nelems(node->output) != s3h_nelems(in))
		return 0;
	const int cols = in->dims[in->n_dims - 1];
	if (cols <= 0)
		return 0;
	for (int k = 1; k < node->n_inputs && k < 3; k++) {
		const struct sam3_tensor *t = node->inputs[k];
		if (t && (t->dtype != in->dtype || s3h_nelems(t) < cols))
			return 0;
	}
	return 1;
}

enum sam3_error s3h_layernorm(const struct sam3_node *node, void *stream)
{
	if (node->n_inputs < 1 || !node->inputs[0] || !node->output) {
		s3h_error("layernorm: NULL tensor");
		return SAM3_EINVAL;
	}
	const struct sam3_tensor *in = node->inputs[0];
	if (!is_float_dtype(in->dtype)) {
		s3h_error("layernorm: unsupported dtype %d", in->dtype);
		return SAM3_EDTYPE;
	}
	if (!s3h_layernorm_ok(node)) {
		s3h_error("layernorm: output, gamma or beta does not match the input");
		return SAM3_EINVAL;
	}
	const int cols = in->dims[in->n_dims - 1];
	const void *g = node->n_inputs > 1 && node->inputs[1] ? node->inputs[1]->data : NULL;
	const void *b = node->n_inputs > 2 && node->inputs[2] ? node->inputs[2]->data : NULL;
	return s3h_hip(s3k_layernorm(in->dtype, in->data, g, b, node->output->data,
				     s3h_nelems(in) / cols, cols, stream),
		       "layernorm");
}

/* ROPE (cpu_rope.c:35-108 and its bf16/f16 twins): x [batch, seq, heads,
 * hd] (F32, F16 or BF16), cos and sin F32 [seq, hd/2]. */
int s3h_rope_ok(const struct sam3_node *node)
{
	if (node->n_inputs < 3 || !node->inputs[0] || !node->inputs[1] || !node->inputs[2] ||
	    !node->output)
		return 0;
	const struct sam3_tensor *x = node->inputs[0], *c = node->inputs[1], *s = node->inputs[2];
	if (!is_float_dtype(x->dtype) || x->n_dims != 4 || (x->dims[3] & 1) ||
	    c->dtype != SAM3_DTYPE_F32 || s->dtype != SAM3_DTYPE_F32 ||
	    node->output->dtype != x->dtype || s3h_nelems(node->output) != s3h_nelems(x))
		return 0;
	const int seq = x->dims[1], half = x->dims[3] / 2;
	return c->n_dims == 2 && c->dims[0] == seq && c->dims[1] == half && s->n_dims == 2 &&
	       s->dims[0] == seq && s->dims[1] == half;
}

enum sam3_error s3h_rope(const struct sam3_node *node, void *stream)
{
	if (node->n_inputs < 3 || !node->inputs[0] || !node->inputs[1] || !node->inputs[2] ||
	    !node->output) {
		s3h_error("rope: NULL tensor");
		return SAM3_EINVAL;
	}
	const struct sam3_tensor *x = node->inputs[0];
	if (!is_float_dtype(x->dtype) || node->inputs[1]->dtype != SAM3_DTYPE_F32 ||
	    node->inputs[2]->dtype != SAM3_DTYPE_F32) {
		s3h_error("rope: input must be F32/F16/BF16 and cos/sin F32");
		return SAM3_EDTYPE;
	}
	if (!s3h_rope_ok(node)) {
		s3h_error("rope: need x [batch, seq, heads, hd] (hd even) and cos/sin [seq, hd/2]");
		return SAM3_EINVAL;
	}
	return s3h_hip(s3k_rope(x->dtype, x->data, (const float *)node->inputs[1]->data,
				(const float *)node->inputs[2]->data, node->output->data, x->dims[0],
				x->dims[1], x->dims[2], x->dims[3], stream),
		       "rope");
}

/* SLICE (cpu_slice.c:19-88): params axis, start, end; one strided copy. */
int s3h_slice_ok(const struct sam3_node *node)
{
	if (node->n_inputs < 1 || !node->inputs[0] || !node->output)
		return 0;
	const struct sam3_tensor *in = node->inputs[0];
	const int axis = node->params[0], start = node->params[1], end = node->params[2];
	return s3h_dtype_size(in->dtype) != 0 && axis >= 0 && axis < in->n_dims && start >= 0 &&
	       end <= in->dims[axis] && start < end && node->output->n_dims > axis &&
	       node->output->dims[axis] == end - start;
}

enum sam3_error s3h_slice(const struct sam3_node *node, void *stream)
{
	if (node->n_inputs < 1 || !node->inputs[0] || !node->output) {
		s3h_error("slice: NULL tensor");
		return SAM3_EINVAL;
	}
	const struct sam3_tensor *in = node->inputs[0];
	const size_t es = s3h_dtype_size(in->dtype);
	if (!es) {
		s3h_error("slice: dtype %d has no element size", in->dtype);
		return SAM3_EDTYPE;
	}
	if (!s3h_slice_ok(node)) {
		s3h_error("slice: invalid axis or range [%d, %d)", node->params[1], node->params[2]);
		return SAM3_EINVAL;
	}
	const int axis = node->params[0], start = node->params[1], end = node->params[2];
	size_t outer = 1, inner = 1;
	for (int d = 0; d < axis; d++)
		outer *= (size_t)in->dims[d];
	for (int d = axis + 1; d < in->n_dims; d++)
		inner *= (size_t)in->dims[d];
	const size_t width = (size_t)(end - start) * inner * es;
	const size_t spitch = (size_t)in->dims[axis] * inner * es;
	if (!outer || !width)
		return SAM3_OK;
	return s3h_hip(hipMemcpy2DAsync(node->output->data, width,
					(const char *)in->data + (size_t)start * inner * es, spitch,
					width, outer, hipMemcpyDeviceToDevice, (hipStream_t)stream),
		       "slice");
}

/* RESHAPE (cpu_reshape.c:19-42): a view. The output takes the input's
 * data pointer and row-major strides; nothing is copied. */
enum sam3_error s3h_reshape(const struct sam3_node *node)
{
	if (node->n_inputs < 1 || !node->inputs[0] || !node->output) {
		s3h_error("reshape: NULL tensor");
		return SAM3_EINVAL;
	}
	const struct sam3_tensor *in = node->inputs[0];
	struct sam3_tensor *out = node->output;
	if (s3h_nelems(in) != s3h_nelems(out)) {
		s3h_error("reshape: element count mismatch %lld != %lld", s3h_nelems(in),
			  s3h_nelems(out));
		return SAM3_EINVAL;
	}
	out->data = in->data;
	out->nbytes = in->nbytes;
	int st = 1;
	for (int i = out->n_dims - 1; i >= 0; i--) {
		out->strides[i] = st;
		st *= out->dims[i];
	}
	return SAM3_OK;
}

/* ------------------------------------------------------------------ */
/* CONV2D and BIAS_ADD                                                  */
/* ------------------------------------------------------------------ */

/* CONV2D as cpu_kernel_conv2d reads it (cpu_conv2d.c:296-368): input
 * [N,H,W,C], weight OHWI [OC,KH,KW,C/groups], output [N,OH,OW,OC] with OH,
 * OW taken from the output; params stride (<= 0 -> 1), pad_h, groups
 * (<= 0 -> 1), pad_w (0 -> pad_h). Same dtype for input, weight and
 * output (cpu_dispatch.c:643-655). */
static enum sam3_error conv_shape(const struct sam3_node *node, struct s3k_conv *c, int quiet)
{
#define CONV_FAIL(code, ...)                    \
	do {                                    \
		if (!quiet)                     \
			s3h_error(__VA_ARGS__); \
		return code;                    \
	} while (0)
	if (!node || node->n_inputs < 2 || !node->inputs[0] || !node->inputs[1] || !node->output)
		CONV_FAIL(SAM3_EINVAL, "conv2d: NULL tensor");
	const struct sam3_tensor *x = node->inputs[0], *w = node->inputs[1], *y = node->output;
	if (!is_float_dtype(x->dtype) || w->dtype != x->dtype || y->dtype != x->dtype)
		CONV_FAIL(SAM3_EDTYPE, "conv2d: input, weight and output must share one of F32/F16/BF16 "
				       "(got %d, %d, %d)", x->dtype, w->dtype, y->dtype);
	if (x->n_dims != 4 || w->n_dims != 4 || y->n_dims != 4)
		CONV_FAIL(SAM3_EINVAL, "conv2d: expected 4D tensors");
	memset(c, 0, sizeof(*c));
	c->kind = x->dtype;
	c->x = x->data;
	c->w = w->data;
	c->y = y->data;
	c->N = x->dims[0];
	c->H = x->dims[1];
	c->W = x->dims[2];
	c->C = x->dims[3];
	c->OC = w->dims[0];
	c->KH = w->dims[1];
	c->KW = w->dims[2];
	c->stride = node->params[0] > 0 ? node->params[0] : 1;
	c->pad_h = node->params[1];
	c->groups = node->params[2] > 0 ? node->params[2] : 1;
	c->pad_w = node->params[3] ? node->params[3] : c->pad_h;
	c->OH = y->dims[1];
	c->OW = y->dims[2];
	if (w->dims[3] * c->groups != c->C)
		CONV_FAIL(SAM3_EINVAL, "conv2d: channel mismatch %d*%d != %d", w->dims[3], c->groups,
			  c->C);
	if (c->C % c->groups || c->OC % c->groups)
		CONV_FAIL(SAM3_EINVAL, "conv2d: channels not divisible by groups");
	if (y->dims[0] != c->N || y->dims[3] != c->OC)
		CONV_FAIL(SAM3_EINVAL, "conv2d: output shape mismatch");
	if (c->N <= 0 || c->H <= 0 || c->W <= 0 || c->C <= 0 || c->OC <= 0 || c->KH <= 0 ||
	    c->KW <= 0 || c->OH <= 0 || c->OW <= 0)
		CONV_FAIL(SAM3_EINVAL, "conv2d: empty dimension");
	if ((long long)c->N * c->H * c->W * c->C > INT32_MAX ||
	    (long long)c->N * c->OH * c->OW * c->OC > INT32_MAX ||
	    (long long)c->OC * c->KH * c->KW * (c->C / c->groups) > INT32_MAX)
		CONV_FAIL(SAM3_EINVAL, "conv2d: tensor of more than 2^31 elements");
	return SAM3_OK;
#undef CONV_FAIL
}

static int conv_f32_split_allowed(void)
{
	return s3h_settings()->f32_split;
}

/* Whether the implicit GEMM (1) or the column matrix + GEMM (2) can run
 * c: groups 1, f32 only with the split allowed, buffer ranges under 2 GiB
 * (and for 1: C % 64 == 0, 16-byte aligned x and w). */
static int conv_implicit_ok(const struct s3k_conv *c)
{
	const int f32 = c->kind == SAM3_DTYPE_F32;
	const long long K = (long long)c->KH * c->KW * c->C;
	const long long pp = f32 ? 3LL * c->C : c->C;
	return c->groups == 1 && (!f32 || conv_f32_split_allowed()) && c->C % 64 == 0 &&
	       !(((uintptr_t)c->x | (uintptr_t)c->w) & 15u) &&
	       (long long)c->N * c->H * c->W * pp * 2 <= 0x7FFFFFF0LL &&
	       (long long)c->OC * K * (f32 ? 3 : 1) * 2 <= 0x7FFFFFF0LL;
}

static int conv_im2col_ok(const struct s3k_conv *c)
{
	const int f32 = c->kind == SAM3_DTYPE_F32;
	const long long M = (long long)c->N * c->OH * c->OW;
	const long long kp = ((long long)c->KH * c->KW * c->C + 7) / 8 * 8 * (f32 ? 3 : 1);
	return c->groups == 1 && (!f32 || conv_f32_split_allowed()) && M * kp * 2 <= 0x7FFFFFF0LL &&
	       (long long)c->OC * kp * 2 <= 0x7FFFFFF0LL && !(((uintptr_t)c->y) & 3u);
}

/* Kernel choice: 1 implicit GEMM, 2 column matrix + GEMM, 3 direct (also
 * for problems under 2^22 multiply-adds, where a GEMM launch does not pay). */
static int conv_path_of(const struct s3k_conv *c)
{
	const long long M = (long long)c->N * c->OH * c->OW;
	const long long K = (long long)c->KH * c->KW * c->C;
	if (M * c->OC * K < (1LL << 22))
		return S3H_CONV_DIRECT;
	if (conv_implicit_ok(c))
		return S3H_CONV_IMPLICIT;
	return conv_im2col_ok(c) ? S3H_CONV_IM2COL : S3H_CONV_DIRECT;
}

static enum sam3_error free_scratch(void *p, void *stream, enum sam3_error err)
{
	if (!p)
		return err;
	enum sam3_error e = s3h_scratch_free(p, stream);
	return err != SAM3_OK ? err : e;
}

/* Conv on device pointers; bias ([OC], the conv's dtype) and GELU are
 * applied in the GEMM epilogue (paths 1 and 2 only). */
static enum sam3_error conv_run(struct s3k_conv *c, int path, void *stream)
{
	const int f32 = c->kind == SAM3_DTYPE_F32;
	const int K = c->KH * c->KW * c->C;
	enum sam3_error err = SAM3_OK;
	if (path == S3H_CONV_DIRECT) {
		if (c->flags) {
			s3h_error("conv2d: the direct kernel has no fused epilogue");
			return SAM3_EINVAL;
		}
		return s3h_hip(s3k_conv_direct(c, stream), "conv2d direct");
	}
	if (path == S3H_CONV_IMPLICIT) {
		if (!f32)
			return s3h_hip(s3k_conv_implicit(c, c->x, c->w, c->C, stream), "conv2d implicit");
		const long long pix = (long long)c->N * c->H * c->W;
		void *xp = NULL, *wp = NULL;
		int own_w = 0;
		err = s3h_scratch_alloc(&xp, (size_t)pix * 3 * c->C * 2, stream);
		if (err == SAM3_OK)
			err = prep_weight(c->w, (size_t)c->OC * K * 4, S3H_PREP_SPLIT_W, c->OC, K, K,
					  (size_t)c->OC * 3 * K * 2, S3K_F32, prep_split_w, stream, &wp, &own_w);
		if (err == SAM3_OK)
			err = s3h_hip(s3k_split3_bf16((const float *)c->x, xp, (int)pix, c->C, c->C, 0, stream),
				      "conv2d split x");
		if (err == SAM3_OK)
			err = s3h_hip(s3k_conv_implicit(c, xp, wp, 3 * c->C, stream), "conv2d implicit");
		return free_scratch(xp, stream, free_scratch(own_w ? wp : NULL, stream, err));
	}
	/* path 2: column matrix [M, Kp] (or planes [M, 3Kp]) and the NT GEMM */
	const int Kp = (K + 7) / 8 * 8, segs = f32 ? 3 : 1;
	const long long M = (long long)c->N * c->OH * c->OW;
	void *col = NULL, *wq = NULL;
	int own_w = 0;
	err = s3h_scratch_alloc(&col, (size_t)M * Kp * segs * 2, stream);
	if (err == SAM3_OK)
		err = prep_weight(c->w, (size_t)c->OC * K * (f32 ? 4 : 2),
				  f32 ? S3H_PREP_PAD_PLANES : S3H_PREP_PAD16, c->OC, K, Kp,
				  (size_t)c->OC * Kp * segs * 2, c->kind, prep_conv_w, stream, &wq, &own_w);
	if (err == SAM3_OK)
		err = s3h_hip(s3k_conv_im2col(c, col, Kp, stream), "conv2d im2col");
	if (err == SAM3_OK) {
		struct s3k_gemm g;
		memset(&g, 0, sizeof(g));
		g.a = col;
		g.b = wq;
		g.c = c->y;
		g.bias = c->bias;
		g.M = (int)M;
		g.N = c->OC;
		g.K = Kp * segs;
		g.lda = g.ldb = Kp * segs;
		g.ldc = c->OC;
		g.batch = 1;
		g.a_kind = g.b_kind = f32 ? S3K_BF16 : c->kind;
		g.c_kind = c->kind;
		g.flags = S3K_B_NT | (c->flags & (S3K_EPI_BIAS | S3K_EPI_GELU));
		err = s3h_hip(s3k_gemm_launch_path(&g, S3K_PATH_MFMA, stream), "conv2d gemm");
	}
	return free_scratch(col, stream, free_scratch(own_w ? wq : NULL, stream, err));
}

int s3h_conv2d_ok(const struct sam3_node *node)
{
	struct s3k_conv c;
	return conv_shape(node, &c, 1) == SAM3_OK;
}

int s3h_conv2d_path(const struct sam3_node *node)
{
	struct s3k_conv c;
	return conv_shape(node, &c, 1) == SAM3_OK ? conv_path_of(&c) : 0;
}

enum sam3_error s3h_conv2d(const struct sam3_node *node, const void *bias, int flags, int path,
			   void *stream)
{
	struct s3k_conv c;
	enum sam3_error err = conv_shape(node, &c, 0);
	if (err != SAM3_OK)
		return err;
	if (path == 0)
		path = conv_path_of(&c);
	if (path < S3H_CONV_IMPLICIT || path > S3H_CONV_DIRECT ||
	    (path == S3H_CONV_IMPLICIT && !conv_implicit_ok(&c)) ||
	    (path == S3H_CONV_IM2COL && !conv_im2col_ok(&c))) {
		s3h_error("conv2d: path %d cannot run this problem", path);
		return SAM3_EINVAL;
	}
	c.bias = bias;
	c.flags = flags & (S3K_EPI_BIAS | S3K_EPI_GELU);
	if ((c.flags & S3K_EPI_BIAS) && !bias) {
		s3h_error("conv2d: NULL bias");
		return SAM3_EINVAL;
	}
	return conv_run(&c, path, stream);
}

enum sam3_error sam3_hip_kernel_conv2d(const struct sam3_node *node, void *stream)
{
	return s3h_conv2d(node, NULL, 0, 0, stream);
}

enum sam3_error sam3_hip_conv2d_on_path(int path, const struct sam3_node *node, void *stream)
{
	return s3h_conv2d(node, NULL, 0, path, stream);
}

int sam3_hip_conv2d_path(const struct sam3_node *node)
{
	return s3h_conv2d_path(node);
}

/* BIAS_ADD (cpu_bias_add.c:65-101, :150-190): x [.., C] + bias [C], F32
 * and BF16 in the reference; F16 as well here. */
int s3h_bias_add_ok(const struct sam3_node *node)
{
	if (!node || node->n_inputs < 2 || !node->inputs[0] || !node->inputs[1] || !node->output)
		return 0;
	const struct sam3_tensor *x = node->inputs[0], *b = node->inputs[1];
	if (!is_float_dtype(x->dtype) || b->dtype != x->dtype || node->output->dtype != x->dtype ||
	    x->n_dims < 1 || s3h_nelems(node->output) != s3h_nelems(x))
		return 0;
	const int C = x->dims[x->n_dims - 1];
	return C > 0 && s3h_nelems(b) == C;
}

enum sam3_error s3h_bias_add(const struct sam3_node *node, void *stream)
{
	if (!node || node->n_inputs < 2 || !node->inputs[0] || !node->inputs[1] || !node->output) {
		s3h_error("bias_add: NULL tensor");
		return SAM3_EINVAL;
	}
	const struct sam3_tensor *x = node->inputs[0];
	if (!is_float_dtype(x->dtype) || node->inputs[1]->dtype != x->dtype) {
		s3h_error("bias_add: x and bias must share one of F32/F16/BF16");
		return SAM3_EDTYPE;
	}
	if (!s3h_bias_add_ok(node)) {
		s3h_error("bias_add: bias must have the last dim's size, output the input's");
		return SAM3_EINVAL;
	}
	const int C = x->dims[x->n_dims - 1];
	return s3h_hip(s3k_bias_add(x->dtype, x->data, node->inputs[1]->data, node->output->data,
				    s3h_nelems(x) / C, C, stream),
		       "bias_add");
}

enum sam3_error sam3_hip_kernel_bias_add(const struct sam3_node *node, void *stream)
{
	return s3h_bias_add(node, stream);
}

/* CONV_TRANSPOSE2D as cpu_kernel_conv_transpose2d reads it
 * (cpu_conv_transpose2d.c:140-217): x [N,H,W,C], w OHWI [OC,KH,KW,C],
 * y [N,OH,OW,OC] with OH = (H-1)*stride - 2*pad + KH (the output must
 * have that shape); params stride (<= 0 -> 1), pad; F32 only
 * (cpu_dispatch.c:553-555). */
struct convt_shape {
	const float *x, *w;
	float *y;
	int N, H, W, C, OC, KH, KW, stride, pad, OH, OW;
};

static enum sam3_error convt_shape(const struct sam3_node *node, struct convt_shape *c, int quiet)
{
#define CT_FAIL(code, ...)                      \
	do {                                    \
		if (!quiet)                     \
			s3h_error(__VA_ARGS__); \
		return code;                    \
	} while (0)
	if (!node || node->n_inputs < 2 || !node->inputs[0] || !node->inputs[1] || !node->output)
		CT_FAIL(SAM3_EINVAL, "conv_transpose2d: NULL tensor");
	const struct sam3_tensor *x = node->inputs[0], *w = node->inputs[1], *y = node->output;
	if (x->dtype != SAM3_DTYPE_F32 || w->dtype != SAM3_DTYPE_F32 || y->dtype != SAM3_DTYPE_F32)
		CT_FAIL(SAM3_EDTYPE, "conv_transpose2d: F32 only (got %d, %d, %d)", x->dtype, w->dtype,
			y->dtype);
	if (x->n_dims != 4 || w->n_dims != 4 || y->n_dims != 4)
		CT_FAIL(SAM3_EINVAL, "conv_transpose2d: expected 4D tensors");
	memset(c, 0, sizeof(*c));
	c->x = x->data;
	c->w = w->data;
	c->y = y->data;
	c->N = x->dims[0];
	c->H = x->dims[1];
	c->W = x->dims[2];
	c->C = x->dims[3];
	c->OC = w->dims[0];
	c->KH = w->dims[1];
	c->KW = w->dims[2];
	c->stride = node->params[0] > 0 ? node->params[0] : 1;
	c->pad = node->params[1];
	if (w->dims[3] != c->C)
		CT_FAIL(SAM3_EINVAL, "conv_transpose2d: channel mismatch %d != %d", w->dims[3], c->C);
	c->OH = (c->H - 1) * c->stride - 2 * c->pad + c->KH;
	c->OW = (c->W - 1) * c->stride - 2 * c->pad + c->KW;
	if (y->dims[0] != c->N || y->dims[1] != c->OH || y->dims[2] != c->OW || y->dims[3] != c->OC)
		CT_FAIL(SAM3_EINVAL, "conv_transpose2d: output shape mismatch");
	if (c->N <= 0 || c->H <= 0 || c->W <= 0 || c->C <= 0 || c->OC <= 0 || c->KH <= 0 ||
	    c->KW <= 0 || c->OH <= 0 || c->OW <= 0 ||
	    (long long)c->N * c->OH * c->OW * c->OC > INT32_MAX ||
	    (long long)c->N * c->H * c->W * c->C > INT32_MAX)
		CT_FAIL(SAM3_EINVAL, "conv_transpose2d: empty or oversized tensor");
	return SAM3_OK;
#undef CT_FAIL
}

static int convt_gemm_ok(const struct convt_shape *c)
{
	const long long M = (long long)c->N * c->H * c->W, T = (long long)c->KH * c->KW;
	return c->stride == c->KH && c->stride == c->KW && c->pad == 0 && c->C % 8 == 0 &&
	       !(((uintptr_t)c->x | (uintptr_t)c->w | (uintptr_t)c->y) & 15u) &&
	       M * T * c->OC * 4 <= 0x7FFFFFF0LL && T * c->OC * c->C * 4 <= 0x7FFFFFF0LL;
}

static int convt_path_of(const struct convt_shape *c)
{
	const long long macs = (long long)c->N * c->H * c->W * c->KH * c->KW * c->OC * c->C;
	return convt_gemm_ok(c) && macs >= (1LL << 22) ? S3H_CONVT_GEMM : S3H_CONVT_DIRECT;
}

int s3h_conv_transpose2d_ok(const struct sam3_node *node)
{
	struct convt_shape c;
	return convt_shape(node, &c, 1) == SAM3_OK;
}

int s3h_conv_transpose2d_path(const struct sam3_node *node)
{
	struct convt_shape c;
	return convt_shape(node, &c, 1) == SAM3_OK ? convt_path_of(&c) : 0;
}

/* OHWI [OC, taps, C] -> [taps * OC, C]: row t*OC + oc is tap t of filter oc */
static int prep_convt_w(const void *w, void *out, int rows, int k, int k_out, int kind, void *stream)
{
	(void)kind;
	const int dims[3] = {rows, k_out, k}, axes[3] = {1, 0, 2};
	return s3k_permute(4, w, out, 3, dims, axes, stream);
}

enum sam3_error s3h_conv_transpose2d(const struct sam3_node *node, const void *bias, int flags,
				     int path, void *stream)
{
	struct convt_shape c;
	enum sam3_error err = convt_shape(node, &c, 0);
	if (err != SAM3_OK)
		return err;
	if (path == 0)
		path = convt_path_of(&c);
	if (path == S3H_CONVT_DIRECT) {
		if (flags) {
			s3h_error("conv_transpose2d: the direct kernel has no fused epilogue");
			return SAM3_EINVAL;
		}
		return s3h_hip(s3k_conv_transpose_direct(c.x, c.w, c.y, c.N, c.H, c.W, c.C, c.OC, c.KH,
							 c.KW, c.stride, c.pad, c.OH, c.OW, stream),
			       "conv_transpose2d direct");
	}
	if (path != S3H_CONVT_GEMM || !convt_gemm_ok(&c)) {
		s3h_error("conv_transpose2d: path %d cannot run this problem", path);
		return SAM3_EINVAL;
	}
	if ((flags & S3K_EPI_BIAS) && !bias) {
		s3h_error("conv_transpose2d: NULL bias");
		return SAM3_EINVAL;
	}
	/* Each input pixel times W' [taps*OC, C] gives its taps' output
	 * pixels: tmp [N*H*W, taps*OC], then [N*H, W, KH, KW*OC] ->
	 * [N*H, KH, W, KW*OC] is y. */
	const int T = c.KH * c.KW, M = c.N * c.H * c.W, NN = T * c.OC;
	void *wt = NULL, *tmp = NULL, *b4 = NULL;
	int own_w = 0;
	err = prep_weight(c.w, (size_t)c.OC * T * c.C * 4, S3H_PREP_CONVT_W, c.OC, c.C, T,
			  (size_t)NN * c.C * 4, S3K_F32, prep_convt_w, stream, &wt, &own_w);
	if (err == SAM3_OK)
		err = s3h_scratch_alloc(&tmp, (size_t)M * NN * 4, stream);
	if (err == SAM3_OK && (flags & S3K_EPI_BIAS)) {
		err = s3h_scratch_alloc(&b4, (size_t)NN * 4, stream);
		if (err == SAM3_OK)
			err = s3h_hip(s3k_repeat_f32((const float *)bias, b4, c.OC, T, stream),
				      "conv_transpose2d bias");
	}
	if (err == SAM3_OK)
		err = matmul_impl(0, SAM3_DTYPE_F32, c.x, SAM3_DTYPE_F32, wt, SAM3_DTYPE_F32, tmp, M, NN,
				  c.C, b4, (flags & (S3K_EPI_BIAS | S3K_EPI_GELU)) | SAM3_HIP_B_NT, stream);
	if (err == SAM3_OK) {
		const int dims[4] = {c.N * c.H, c.W, c.KH, c.KW * c.OC}, axes[4] = {0, 2, 1, 3};
		err = s3h_hip(s3k_permute(4, tmp, c.y, 4, dims, axes, stream), "conv_transpose2d shuffle");
	}
	err = free_scratch(b4, stream, err);
	err = free_scratch(tmp, stream, err);
	return free_scratch(own_w ? wt : NULL, stream, err);
}

enum sam3_error sam3_hip_kernel_conv_transpose2d(const struct sam3_node *node, void *stream)
{
	return s3h_conv_transpose2d(node, NULL, 0, 0, stream);
}

enum sam3_error sam3_hip_conv_transpose2d_on_path(int path, const struct sam3_node *node,
						  void *stream)
{
	return s3h_conv_transpose2d(node, NULL, 0, path, stream);
}

int sam3_hip_conv_transpose2d_path(const struct sam3_node *node)
{
	return s3h_conv_transpose2d_path(node);
}

/* MAXPOOL2D as cpu_kernel_maxpool2d reads it (cpu_maxpool2d.c:113-177):
 * params kernel (<= 0 -> 2), stride (<= 0 -> kernel); OH = (H - kernel)
 * / stride + 1; F32 only (cpu_dispatch.c:556-558). */
static enum sam3_error maxpool_shape(const struct sam3_node *node, int *k, int *st, int quiet)
{
	if (!node || node->n_inputs < 1 || !node->inputs[0] || !node->output) {
		if (!quiet)
			s3h_error("maxpool2d: NULL tensor");
		return SAM3_EINVAL;
	}
	const struct sam3_tensor *x = node->inputs[0], *y = node->output;
	if (x->dtype != SAM3_DTYPE_F32 || y->dtype != SAM3_DTYPE_F32) {
		if (!quiet)
			s3h_error("maxpool2d: F32 only");
		return SAM3_EDTYPE;
	}
	*k = node->params[0] > 0 ? node->params[0] : 2;
	*st = node->params[1] > 0 ? node->params[1] : *k;
	const int OH = x->n_dims == 4 ? (x->dims[1] - *k) / *st + 1 : 0;
	const int OW = x->n_dims == 4 ? (x->dims[2] - *k) / *st + 1 : 0;
	if (x->n_dims != 4 || y->n_dims != 4 || x->dims[1] < *k || x->dims[2] < *k ||
	    y->dims[0] != x->dims[0] || y->dims[1] != OH || y->dims[2] != OW ||
	    y->dims[3] != x->dims[3]) {
		if (!quiet)
			s3h_error("maxpool2d: expected 4D tensors and output [N, OH, OW, C]");
		return SAM3_EINVAL;
	}
	return SAM3_OK;
}

int s3h_maxpool2d_ok(const struct sam3_node *node)
{
	int k, st;
	return maxpool_shape(node, &k, &st, 1) == SAM3_OK;
}

enum sam3_error s3h_maxpool2d(const struct sam3_node *node, void *stream)
{
	int k, st;
	enum sam3_error err = maxpool_shape(node, &k, &st, 0);
	if (err != SAM3_OK)
		return err;
	const struct sam3_tensor *x = node->inputs[0], *y = node->output;
	return s3h_hip(s3k_maxpool2d(x->data, y->data, x->dims[0], x->dims[1], x->dims[2], x->dims[3], k,
				     st, y->dims[1], y->dims[2], stream),
		       "maxpool2d");
}

enum sam3_error sam3_hip_kernel_maxpool2d(const struct sam3_node *node, void *stream)
{
	return s3h_maxpool2d(node, stream);
}

enum sam3_error sam3_hip_kernel_layernorm(const struct sam3_node *node, void *stream)
{
	return node ? s3h_layernorm(node, stream) : (s3h_error("layernorm: NULL node"), SAM3_EINVAL);
}

enum sam3_error sam3_hip_kernel_rope(const struct sam3_node *node, void *stream)
{
	return node ? s3h_rope(node, stream) : (s3h_error("rope: NULL node"), SAM3_EINVAL);
}

enum sam3_error sam3_hip_kernel_slice(const struct sam3_node *node, void *stream)
{
	return node ? s3h_slice(node, stream) : (s3h_error("slice: NULL node"), SAM3_EINVAL);
}

enum sam3_error sam3_hip_kernel_transpose(const struct sam3_node *node, void *stream)
{
	return node ? s3h_transpose(node, stream) : (s3h_error("transpose: NULL node"), SAM3_EINVAL);
}

enum sam3_error sam3_hip_kernel_reshape(const struct sam3_node *node)
{
	return node ? s3h_reshape(node) : (s3h_error("reshape: NULL node"), SAM3_EINVAL);
}

/* Shapes as cpu_kernel_sdpa reads them (cpu_sdpa.c:216-288): 4-D
 * [B, H, seq, hd] or 2-D [seq, hd], head_dim = params[0]. */
static enum sam3_error sdpa_shape(const struct sam3_node *node, int *BH, int *Sq, int *Sk,
				  int *D, int quiet)
{
#define SDPA_FAIL(code, ...)                    \
	do {                                    \
		if (!quiet)                     \
			s3h_error(__VA_ARGS__); \
		return code;                    \
	} while (0)
	if (!node || node->n_inputs < 3 || !node->inputs[0] || !node->inputs[1] ||
	    !node->inputs[2] || !node->output) {
		SDPA_FAIL(SAM3_EINVAL, "sdpa: NULL tensor");
	}
	const struct sam3_tensor *Q = node->inputs[0], *K = node->inputs[1],
				 *V = node->inputs[2], *O = node->output;
	const struct sam3_tensor *M = node->n_inputs > 3 ? node->inputs[3] : NULL;
	const int dt = Q->dtype;
	if (!is_float_dtype(dt) || (int)K->dtype != dt || (int)V->dtype != dt ||
	    (int)O->dtype != dt || (M && M->dtype != SAM3_DTYPE_F32)) {
		SDPA_FAIL(SAM3_EDTYPE, "sdpa: Q, K, V and out need one of F32/F16/BF16, mask F32");
	}
	const int nd = Q->n_dims;
	if ((nd != 2 && nd != 4) || K->n_dims != nd || V->n_dims != nd) {
		SDPA_FAIL(SAM3_EINVAL, "sdpa: tensors must be 2-D [seq, hd] or 4-D [B, H, seq, hd]");
	}
	*D = node->params[0];
	if (nd == 4) {
		*BH = Q->dims[0] * Q->dims[1];
		*Sq = Q->dims[2];
		*Sk = K->dims[2];
	} else {
		*BH = 1;
		*Sq = Q->dims[0];
		*Sk = K->dims[0];
	}
	const long long nq = (long long)*BH * *Sq * *D, nk = (long long)*BH * *Sk * *D;
	if (*D <= 0 || s3h_nelems(Q) < nq || s3h_nelems(O) < nq || s3h_nelems(K) < nk ||
	    s3h_nelems(V) < nk || (M && s3h_nelems(M) < (long long)*Sq * *Sk)) {
		SDPA_FAIL(SAM3_EINVAL, "sdpa: tensor sizes do not match head_dim %d", *D);
	}
	return SAM3_OK;
#undef SDPA_FAIL
}

int s3h_sdpa_node_ok(const struct sam3_node *node)
{
	int BH, Sq, Sk, D;
	return sdpa_shape(node, &BH, &Sq, &Sk, &D, 1) == SAM3_OK && D <= 512;
}

enum sam3_error sam3_hip_kernel_sdpa(const struct sam3_node *node, void *stream)
{
	int BH, Sq, Sk, D;
	enum sam3_error err = sdpa_shape(node, &BH, &Sq, &Sk, &D, 0);
	if (err != SAM3_OK)
		return err;
	const struct sam3_tensor *M = node->n_inputs > 3 ? node->inputs[3] : NULL;
	return sam3_hip_sdpa(node->inputs[0]->dtype, node->inputs[0]->data, node->inputs[1]->data,
			     node->inputs[2]->data, M ? (const float *)M->data : NULL,
			     node->output->data, BH, Sq, Sk, D, stream);
}

/* The SDPA node (4-D [B, H, Sq, D]) with its output stored head-merged
 * at `out`: [B, Sq, H, D], what TRANSPOSE (0,2,1,3) of its output
 * gives, as f32 (S3H_A_PLAIN) or as the operand form fmt of a GEMM
 * reading rows of H*D (f32 SDPA on the MFMA kernel). Inputs read from
 * the node's tensors' data (device addresses). */
enum sam3_error s3h_sdpa_merged(const struct sam3_node *node, void *out, int fmt, unsigned *ovf,
				unsigned ovf_tag, void *stream)
{
	int BH, Sq, Sk, D;
	enum sam3_error err = sdpa_shape(node, &BH, &Sq, &Sk, &D, 0);
	if (err != SAM3_OK)
		return err;
	const struct sam3_tensor *Q = node->inputs[0];
	if (Q->n_dims != 4 || !out) {
		s3h_error("sdpa: head-merged output needs 4-D tensors");
		return SAM3_EINVAL;
	}
	const struct sam3_tensor *M = node->n_inputs > 3 ? node->inputs[3] : NULL;
	const int dt = Q->dtype;
	if (!s3k_attn_path(dt, Q->data, node->inputs[1]->data, node->inputs[2]->data, out, BH, Sq,
			   Sk, D)) {
		s3h_error("sdpa: no kernel for D=%d", D);
		return SAM3_EINVAL;
	}
	const int ofmt = fmt == S3H_A_PLANES ? S3K_LN_PLANES : fmt == S3H_A_F16 ? S3K_LN_F16 : 0;
	if (fmt != S3H_A_PLAIN && !ofmt) {
		s3h_error("sdpa: unknown output form %d", fmt);
		return SAM3_EINVAL;
	}
	return s3h_hip(s3k_attn_heads(0, dt, Q->data, node->inputs[1]->data, node->inputs[2]->data,
				      M ? (const float *)M->data : NULL, out, BH, Sq, Sk, D,
				      Q->dims[1], ofmt, ovf, ovf_tag, stream),
		       "sdpa (heads merged)");
}

enum sam3_error sam3_hip_dispatch_node(const struct sam3_node *node, void *stream)
{
	if (!node) {
		s3h_error("hip_dispatch: NULL node");
		return SAM3_EINVAL;
	}
	if (node->op == SAM3_OP_NONE)
		return SAM3_OK;
	if (node->n_inputs < 1 || !node->inputs[0]) {
		s3h_error("hip_dispatch: node op=%d has no inputs", node->op);
		return SAM3_EINVAL;
	}
	/* Q, K, V share a dtype and the mask is F32 (checked by the kernel);
	 * ROPE takes F32 cos/sin with any float input (cpu_dispatch.c:618-640);
	 * RESHAPE is a view of any dtype */
	if (node->op == SAM3_OP_SDPA)
		return sam3_hip_kernel_sdpa(node, stream);
	if (node->op == SAM3_OP_ROPE)
		return s3h_rope(node, stream);
	if (node->op == SAM3_OP_RESHAPE)
		return s3h_reshape(node);
	int dtype = node->inputs[0]->dtype;
	const int mixed_q8 = node->op == SAM3_OP_MATMUL && node->n_inputs >= 2 &&
			     node->inputs[1] && node->inputs[1]->dtype == SAM3_DTYPE_Q8_0 &&
			     dtype == SAM3_DTYPE_F32;
	if (mixed_q8) {
		dtype = SAM3_DTYPE_Q8_0;
	} else {
		for (int i = 1; i < node->n_inputs; i++) {
			if (node->inputs[i] && (int)node->inputs[i]->dtype != dtype) {
				s3h_error("hip_dispatch: dtype mismatch input[0]=%d input[%d]=%d",
					  dtype, i, node->inputs[i]->dtype);
				return SAM3_EDTYPE;
			}
		}
	}
	if ((unsigned)node->op >= (unsigned)SAM3_OP_COUNT ||
	    (unsigned)dtype >= (unsigned)SAM3_DTYPE_COUNT) {
		s3h_error("hip_dispatch: out-of-range op=%d dtype=%d", node->op, dtype);
		return SAM3_EDTYPE;
	}
	switch (node->op) {
	case SAM3_OP_CAST:
		if (is_float_dtype(dtype))
			return sam3_hip_kernel_cast(node, stream);
		break;
	case SAM3_OP_MATMUL:
		switch (dtype) {
		case SAM3_DTYPE_F32:  return sam3_hip_kernel_matmul(node, stream);
		case SAM3_DTYPE_F16:  return sam3_hip_kernel_matmul_f16(node, stream);
		case SAM3_DTYPE_BF16: return sam3_hip_kernel_matmul_bf16(node, stream);
		case SAM3_DTYPE_Q8_0: return sam3_hip_kernel_matmul_q8(node, stream);
		default: break;
		}
		break;
	case SAM3_OP_ADD:
		if (is_float_dtype(dtype))
			return s3h_add(node, stream);
		break;
	case SAM3_OP_GELU:
		if (is_float_dtype(dtype))
			return s3h_gelu(node, stream);
		break;
	case SAM3_OP_TRANSPOSE:
		if (s3h_dtype_size(dtype))
			return s3h_transpose(node, stream);
		break;
	case SAM3_OP_LAYERNORM:
		if (is_float_dtype(dtype))
			return s3h_layernorm(node, stream);
		break;
	case SAM3_OP_SLICE:
		if (s3h_dtype_size(dtype))
			return s3h_slice(node, stream);
		break;
	case SAM3_OP_CONV2D:
		if (is_float_dtype(dtype))
			return s3h_conv2d(node, NULL, 0, 0, stream);
		break;
	case SAM3_OP_BIAS_ADD:
		if (is_float_dtype(dtype))
			return s3h_bias_add(node, stream);
		break;
	case SAM3_OP_CONV_TRANSPOSE2D:
		if (dtype == SAM3_DTYPE_F32)
			return s3h_conv_transpose2d(node, NULL, 0, 0, stream);
		break;
	case SAM3_OP_MAXPOOL2D:
		if (dtype == SAM3_DTYPE_F32)
			return s3h_maxpool2d(node, stream);
		break;
	default:
		break;
	}
	s3h_error("hip_dispatch: no kernel for op=%d dtype=%d", node->op, dtype);
	return SAM3_EDTYPE;
}

/* ------------------------------------------------------------------ */
/* Device helpers                                                       */
/* ------------------------------------------------------------------ */
int sam3_hip_device_count(void)
{
	int n = 0;
	if (hipGetDeviceCount(&n) != hipSuccess)
		return 0;
	return n;
}

enum sam3_error sam3_hip_set_device(int device)
{
	return s3h_hip(hipSetDevice(device), "set_device");
}

enum sam3_error sam3_hip_malloc(void **ptr, size_t nbytes)
{
	if (!ptr) {
		s3h_error("malloc: NULL out pointer");
		return SAM3_EINVAL;
	}
	*ptr = NULL;
	return s3h_hip(hipMalloc(ptr, nbytes ? nbytes : 1), "malloc");
}

enum sam3_error sam3_hip_free(void *ptr)
{
	return s3h_hip(hipFree(ptr), "free");
}

enum sam3_error sam3_hip_memcpy_h2d(void *dst, const void *src, size_t nbytes)
{
	return s3h_hip(hipMemcpy(dst, src, nbytes, hipMemcpyHostToDevice), "memcpy_h2d");
}

enum sam3_error sam3_hip_memcpy_d2h(void *dst, const void *src, size_t nbytes)
{
	return s3h_hip(hipMemcpy(dst, src, nbytes, hipMemcpyDeviceToHost), "memcpy_d2h");
}

enum sam3_error sam3_hip_memcpy_d2d(void *dst, const void *src, size_t nbytes)
{
	return s3h_hip(hipMemcpy(dst, src, nbytes, hipMemcpyDeviceToDevice), "memcpy_d2d");
}

enum sam3_error sam3_hip_synchronize(void)
{
	return s3h_hip(hipDeviceSynchronize(), "synchronize");
}

enum sam3_error sam3_hip_stream_create(void **stream)
{
	if (!stream) {
		s3h_error("stream_create: NULL out pointer");
		return SAM3_EINVAL;
	}
	return s3h_hip(hipStreamCreateWithFlags((hipStream_t *)stream, hipStreamNonBlocking),
		       "stream_create");
}

enum sam3_error sam3_hip_stream_destroy(void *stream)
{
	/* the stream's idle scratch blocks go back to the runtime first: a
	 * later stream may get the same handle while this one's last kernels
	 * still run */
	s3h_scratch_release(stream);
	return s3h_hip(hipStreamDestroy((hipStream_t)stream), "stream_destroy");
}

enum sam3_error sam3_hip_stream_synchronize(void *stream)
{
	return s3h_hip(hipStreamSynchronize((hipStream_t)stream), "stream_synchronize");
}

enum sam3_error sam3_hip_event_create(void **event)
{
	if (!event) {
		s3h_error("event_create: NULL out pointer");
		return SAM3_EINVAL;
	}
	return s3h_hip(hipEventCreate((hipEvent_t *)event), "event_create");
}

enum sam3_error sam3_hip_event_destroy(void *event)
{
	return s3h_hip(hipEventDestroy((hipEvent_t)event), "event_destroy");
}

enum sam3_error sam3_hip_event_record(void *event, void *stream)
{
	return s3h_hip(hipEventRecord((hipEvent_t)event, (hipStream_t)stream), "event_record");
}

enum sam3_error sam3_hip_event_elapsed_ms(float *ms, void *start, void *stop)
{
	if (!ms) {
		s3h_error("event_elapsed: NULL out pointer");
		return SAM3_EINVAL;
	}
	return s3h_hip(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop),
		       "event_elapsed");
}

const char *sam3_hip_device_arch(int device)
{
	static _Thread_local char arch[64];
	hipDeviceProp_t prop;
	arch[0] = 0;
	if (hipGetDeviceProperties(&prop, device) == hipSuccess) {
		strncpy(arch, prop.gcnArchName, sizeof(arch) - 1);
		arch[sizeof(arch) - 1] = 0;
	}
	return arch;
}
