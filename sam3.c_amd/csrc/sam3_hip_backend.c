/*
 * sam3_hip_backend.c - the HIP backend object behind sam3.c's backend
 * vtable (src/backend/backend.h:31-62): init, free, alloc_tensor,
 * graph_eval, arena_reset, cache_invalidate.
 *
 * graph_eval walks g->nodes in order, as cpu_graph_eval does
 * (src/backend/cpu/cpu_backend.c:124-151), and stops at the first failing
 * node. MATMUL runs on the GPU; so do ADD, GELU and last-two-dims
 * TRANSPOSE. Chains the graph builder emits for a linear layer
 * (gh_linear: TRANSPOSE(W) -> MATMUL -> ADD(bias), graph_helpers.c:
 * 297-320) and an MLP (gh_mlp: ... -> GELU, graph_helpers.c:1258-1276)
 * run as one GEMM launch: the transpose becomes the [N,K] weight layout,
 * the bias and GELU the epilogue. The folding applies only when each
 * folded intermediate has exactly one consumer in the graph; folded
 * intermediates are not materialised. Any other op is handed to the host
 * dispatcher (sam3.c's cpu_dispatch_node in an integration), or fails
 * with SAM3_EDTYPE when none is set.
 *
 * Memory. sam3.c tensors point at host memory (the CPU arena or the
 * read-only .sam3 mmap, graph_helpers.c:122-145). Each host buffer gets a
 * device shadow in HBM, tracked by a residency entry {host ptr, device
 * ptr, which copy is current}:
 *   - an input not yet on the device is uploaded once; non-ephemeral
 *     inputs (weights) keep their shadow across graph_eval calls until
 *     cache_invalidate / arena_reset drops it (tensor.h:31-38,
 *     backend.h:50-55);
 *   - outputs are written to the shadow; when the eval ends the graph's
 *     final outputs (node outputs no node consumes) are copied back to
 *     the host, as the reference's GPU backend does, unless
 *     g->no_readback is set; intermediates stay on the device;
 *   - before a host-dispatched node, its inputs are copied back first.
 * Tensors whose data already is device memory are used in place.
 * alloc_tensor hands out pinned host memory (hipHostMalloc), so the
 * copies above run at full PCIe/xGMI rate and asynchronously.
 *
 * Mapped weights. sam3_hip_backend_map_weights copies a whole host range
 * (the data blob of an mmap'd .sam3 file, weight.c:303-474, whose tensors
 * sit at 64-byte aligned offsets) into one HBM allocation in a single
 * staged transfer. Any tensor whose data lies inside a mapped range is
 * then read from that copy at the same offset: no residency entry, no
 * per-tensor upload. Tensors built on the device (sam3_hip_backend_fuse_rows)
 * are owned by the backend until it is destroyed.
 */
#include "sam3_hip.h"
#include "sam3_hip_internal.h"
#include "s3k.h"

#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define S3H_ARENA_DEFAULT (256UL << 20)
#define S3H_ARENA_ALIGN 256

struct s3h_res {
	const char *host;
	size_t nbytes;           /* host bytes of the tensor last bound here:
				  * every host copy moves exactly this many */
	size_t cap;              /* bytes of the device allocation (>= the
				  * tensor, or its GEMM operand form)      */
	void *dev;
	unsigned char dev_valid;
	unsigned char host_valid;
	unsigned char keep;      /* survives the end of this eval            */
	unsigned char produced;  /* written by a GPU node in this eval        */
	unsigned char written;   /* written by a GPU node in any eval         */
	unsigned char fmt;       /* S3H_A_*: the device copy holds a GEMM
				  * operand form, not the tensor's dtype    */
	unsigned char fresh;     /* uploaded from the host in this eval      */
	const void *ln[3];       /* fmt S3H_A_LN: the LayerNorm's input,
				  * gamma and beta on the device (the
				  * consuming GEMM normalizes as it reads) */
	struct s3h_att1_in att;  /* fmt S3H_A_ATT1: the one-key attention's
				  * q, k, v, mask entry, scale and head size
				  * (the consuming GEMV forms its output)  */
};

/* A prepared copy of a constant weight (s3h_prep_*). */
struct s3h_prep {
	const char *src;
	int tag, rows, k;
	void *dev;
	size_t bytes;
};

/* A host range copied to HBM once: [host, host + nbytes) -> dev. */
struct s3h_blob {
	const char *host;
	size_t nbytes;
	char *dev;
};

struct sam3_hip_backend {
	struct sam3_backend base; /* must be first (backend.h:59-62) */
	int device;
	hipStream_t stream;
	struct s3h_res *res;
	int n_res, cap_res;
	/* open-addressing index host address -> res slot + 1 (0 empty),
	 * rebuilt after drops (which move entries) */
	int *res_ix;
	size_t res_ix_cap;
	int res_ix_dirty;
	struct s3h_blob *blobs;
	int n_blobs, cap_blobs;
	void **owned; /* device buffers made by fuse_rows */
	int n_owned, cap_owned;
	struct s3h_prep *prep;
	int n_prep, cap_prep;
	struct s3h_stager stager;
	char *arena;
	size_t arena_size, arena_off;
	sam3_hip_host_dispatch_fn host_fn;
	void *host_ctx;
	struct sam3_hip_eval_stats stats;
	/* f16 GEMM operands written by fused producers: a device word the
	 * writers set to this eval's tag when a value does not fit f16
	 * (then the eval is redone without f16 operand forms) */
	unsigned *ovf;
	unsigned ovf_tag;
	int f16_writes;
	int no_f16_ops;
	/* the row tags of this eval's GEMM-written f16 operands (struct
	 * s3k_gemm rowf), checked together before the flag is read */
	unsigned *rowf[32];
	int rowf_rows[32];
	int n_rowf;
};

/* ------------------------------------------------------------------ */
/* Residency table                                                      */
/* ------------------------------------------------------------------ */
static size_t res_hash(const void *p)
{
	uint64_t x = (uint64_t)(uintptr_t)p;
	x ^= x >> 33;
	x *= 0xff51afd7ed558ccdULL;
	x ^= x >> 33;
	return (size_t)x;
}

static void res_ix_put(struct sam3_hip_backend *hb, int slot)
{
	size_t k = res_hash(hb->res[slot].host) & (hb->res_ix_cap - 1);
	while (hb->res_ix[k])
		k = (k + 1) & (hb->res_ix_cap - 1);
	hb->res_ix[k] = slot + 1;
}

/* (Re)build the index for the current table, at most half full. Returns
 * 0 when out of host memory (lookups then scan the table). */
static int res_ix_rebuild(struct sam3_hip_backend *hb)
{
	size_t cap = 64;
	while (cap < 4 * (size_t)hb->n_res)
		cap <<= 1;
	if (cap != hb->res_ix_cap) {
		int *ix = realloc(hb->res_ix, cap * sizeof(*ix));
		if (!ix)
			return 0;
		hb->res_ix = ix;
		hb->res_ix_cap = cap;
	}
	memset(hb->res_ix, 0, hb->res_ix_cap * sizeof(*hb->res_ix));
	for (int i = 0; i < hb->n_res; i++)
		res_ix_put(hb, i);
	hb->res_ix_dirty = 0;
	return 1;
}

/* The entry for host address `host`. Graphs of several layers hold
 * hundreds of entries and look them up several times per node: a hash
 * index, not a scan. Host addresses are unique in the table. */
static struct s3h_res *res_find(struct sam3_hip_backend *hb, const void *host)
{
	if ((hb->res_ix_dirty || 2 * (size_t)hb->n_res >= hb->res_ix_cap) && !res_ix_rebuild(hb)) {
		for (int i = 0; i < hb->n_res; i++)
			if (hb->res[i].host == host)
				return &hb->res[i];
		return NULL;
	}
	size_t k = res_hash(host) & (hb->res_ix_cap - 1);
	while (hb->res_ix[k]) {
		struct s3h_res *e = &hb->res[hb->res_ix[k] - 1];
		if (e->host == host)
			return e;
		k = (k + 1) & (hb->res_ix_cap - 1);
	}
	return NULL;
}

/* The backend whose graph_eval runs on this thread (prepared weights). */
static _Thread_local struct sam3_hip_backend *s3h_cur;

/* Drop the prepared copies whose source lies in device range [lo, hi),
 * and the copies prepared from those in turn. */
static void prep_drop_range(struct sam3_hip_backend *hb, const char *lo, const char *hi)
{
	for (int i = hb->n_prep - 1; i >= 0 && i < hb->n_prep; i--) {
		if (hb->prep[i].src < lo || hb->prep[i].src >= hi)
			continue;
		const struct s3h_prep p = hb->prep[i];
		hb->prep[i] = hb->prep[hb->n_prep - 1];
		hb->n_prep--;
		prep_drop_range(hb, p.dev, (const char *)p.dev + p.bytes);
		(void)s3h_scratch_free(p.dev, hb->stream);
		i = hb->n_prep;
	}
}

static void res_drop_at(struct sam3_hip_backend *hb, int i)
{
	if (hb->res[i].dev)
		prep_drop_range(hb, hb->res[i].dev, (const char *)hb->res[i].dev + hb->res[i].cap);
	if (hb->res[i].dev)
		(void)s3h_scratch_free(hb->res[i].dev, hb->stream);
	hb->res[i] = hb->res[hb->n_res - 1];
	hb->n_res--;
	hb->res_ix_dirty = 1;
}

static void res_drop_range(struct sam3_hip_backend *hb, const char *lo, const char *hi)
{
	for (int i = hb->n_res - 1; i >= 0; i--) {
		const char *s = hb->res[i].host, *e = s + hb->res[i].nbytes;
		if (s < hi && e > lo)
			res_drop_at(hb, i);
	}
}

/* A new entry for host tensor t with a device allocation of dev_bytes. */
static enum sam3_error res_new(struct sam3_hip_backend *hb, const struct sam3_tensor *t,
			       size_t dev_bytes, struct s3h_res **out)
{
	if (hb->n_res == hb->cap_res) {
		int cap = hb->cap_res ? hb->cap_res * 2 : 256;
		struct s3h_res *r = realloc(hb->res, (size_t)cap * sizeof(*r));
		if (!r) {
			s3h_error("graph_eval: out of host memory for the residency table");
			return SAM3_ENOMEM;
		}
		hb->res = r;
		hb->cap_res = cap;
	}
	struct s3h_res *e = &hb->res[hb->n_res];
	memset(e, 0, sizeof(*e));
	e->host = t->data;
	e->nbytes = s3h_tensor_bytes(t);
	e->cap = dev_bytes;
	enum sam3_error err = s3h_scratch_alloc(&e->dev, dev_bytes, hb->stream);
	if (err != SAM3_OK)
		return err;
	e->host_valid = 1;
	e->keep = !t->ephemeral;
	hb->n_res++;
	if (!hb->res_ix_dirty && 2 * (size_t)hb->n_res < hb->res_ix_cap)
		res_ix_put(hb, hb->n_res - 1);
	else
		hb->res_ix_dirty = 1;
	*out = e;
	return SAM3_OK;
}

/* Device address of [p, p + nbytes) when it lies inside a mapped range. */
static void *blob_addr(const struct sam3_hip_backend *hb, const void *p, size_t nbytes)
{
	const char *c = (const char *)p;
	for (int i = 0; i < hb->n_blobs; i++) {
		const struct s3h_blob *b = &hb->blobs[i];
		if (c >= b->host && c < b->host + b->nbytes && nbytes <= b->nbytes - (size_t)(c - b->host))
			return b->dev + (c - b->host);
	}
	return NULL;
}

static void blob_drop_at(struct sam3_hip_backend *hb, int i)
{
	prep_drop_range(hb, hb->blobs[i].dev, hb->blobs[i].dev + hb->blobs[i].nbytes);
	(void)hipStreamSynchronize(hb->stream);
	(void)hipFree(hb->blobs[i].dev);
	hb->blobs[i] = hb->blobs[hb->n_blobs - 1];
	hb->n_blobs--;
}

static int is_device_ptr(const void *p)
{
	hipPointerAttribute_t attr;
	memset(&attr, 0, sizeof(attr));
	hipError_t e = hipPointerGetAttributes(&attr, p);
	if (e != hipSuccess) {
		(void)hipGetLastError();
		return 0;
	}
	return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

/* Device address of tensor t's data, uploading it if needed. */
static enum sam3_error dev_in(struct sam3_hip_backend *hb, const struct sam3_tensor *t,
			      void **out)
{
	if (!t || !t->data) {
		s3h_error("graph_eval: input tensor without data");
		return SAM3_EINVAL;
	}
	size_t nbytes = s3h_tensor_bytes(t);
	void *mapped = hb->n_blobs ? blob_addr(hb, t->data, nbytes) : NULL;
	if (mapped) {
		*out = mapped;
		hb->stats.mapped_reads++;
		return SAM3_OK;
	}
	/* a residency entry exists only for host memory, so the runtime's
	 * pointer lookup (a few microseconds per call) runs only for
	 * pointers this backend has not seen */
	struct s3h_res *e = res_find(hb, t->data);
	if (!e && is_device_ptr(t->data)) {
		*out = t->data;
		return SAM3_OK;
	}
	if (e && e->fmt) {
		/* a producer wrote the consuming GEMM's operand form */
		*out = e->dev;
		return SAM3_OK;
	}
	/* The same host address may now hold a different tensor (sam3.c
	 * recycles arena memory between graphs without cache_invalidate). A
	 * tensor larger than the one last bound here is a new tensor: its
	 * bytes come from the host, into the shadow if it is big enough. A
	 * smaller one reads the shadow's prefix. */
	if (e && e->cap < nbytes) {
		res_drop_at(hb, (int)(e - hb->res));
		e = NULL;
	} else if (e && e->nbytes < nbytes) {
		e->nbytes = nbytes;
		e->dev_valid = 0;
		e->host_valid = 1;
	}
	if (!e) {
		enum sam3_error err = res_new(hb, t, nbytes, &e);
		if (err != SAM3_OK)
			return err;
	}
	/* an ephemeral input is host data the caller may have rewritten since
	 * the last eval; only a copy a node of this graph wrote is current */
	if (t->ephemeral && !e->produced && !e->fresh)
		e->dev_valid = 0;
	if (!e->dev_valid) {
		e->nbytes = nbytes;
		enum sam3_error err = s3h_hip(hipMemcpyAsync(e->dev, e->host, e->nbytes,
							     hipMemcpyHostToDevice, hb->stream),
					      "graph_eval: upload");
		if (err != SAM3_OK)
			return err;
		e->dev_valid = 1;
		e->fresh = 1;
		hb->stats.uploads++;
	} else if (!e->produced) {
		hb->stats.cache_hits++;
	}
	if (t->ephemeral)
		e->keep = 0;
	*out = e->dev;
	return SAM3_OK;
}

/* Device address the output of a GPU node is written to. */
static enum sam3_error dev_out(struct sam3_hip_backend *hb, const struct sam3_tensor *t,
			       void **out)
{
	if (!t || !t->data) {
		s3h_error("graph_eval: output tensor without data");
		return SAM3_EINVAL;
	}
	struct s3h_res *e = res_find(hb, t->data);
	if (!e && is_device_ptr(t->data)) {
		*out = t->data;
		return SAM3_OK;
	}
	size_t nbytes = s3h_tensor_bytes(t);
	if (e && e->cap < nbytes) {
		res_drop_at(hb, (int)(e - hb->res));
		e = NULL;
	}
	if (!e) {
		enum sam3_error err = res_new(hb, t, nbytes, &e);
		if (err != SAM3_OK)
			return err;
	}
	e->nbytes = nbytes;
	e->dev_valid = 1;
	e->host_valid = 0;
	e->produced = 1;
	e->written = 1;
	e->keep = 1;
	e->fmt = 0;
	*out = e->dev;
	return SAM3_OK;
}

/* A device buffer of nbytes for output t holding the operand form fmt of
 * the one GEMM that reads it: never downloaded, stale after the eval. */
/* The row tags collected so far: rows whose nonzero values were all
 * below 2^-10 set the range flag (s3k_rowflag_check). */
static enum sam3_error rowf_flush(struct sam3_hip_backend *hb)
{
	enum sam3_error err = SAM3_OK;
	if (hb->n_rowf)
		err = s3h_hip(s3k_rowflag_check(hb->n_rowf, hb->rowf, hb->rowf_rows, hb->ovf_tag,
						hb->ovf, hb->stream),
			      "graph_eval: row tag check");
	hb->n_rowf = 0;
	return err;
}

/* *same (when not NULL): the allocation held this operand form before
 * (not new, not another form), so words past the data keep their
 * contents from earlier evals of this form. */
static enum sam3_error dev_out_fmt(struct sam3_hip_backend *hb, const struct sam3_tensor *t,
				   size_t nbytes, int fmt, void **out, int *same)
{
	struct s3h_res *e = res_find(hb, t->data);
	if (e && e->cap < nbytes) {
		res_drop_at(hb, (int)(e - hb->res));
		e = NULL;
	}
	if (same)
		*same = e && e->fmt == fmt;
	if (!e) {
		enum sam3_error err = res_new(hb, t, nbytes, &e);
		if (err != SAM3_OK)
			return err;
	}
	e->nbytes = s3h_tensor_bytes(t);
	e->dev_valid = 1;
	e->host_valid = 0;
	e->produced = 1;
	e->written = 1;
	e->keep = 1;
	e->fmt = (unsigned char)fmt;
	*out = e->dev;
	return SAM3_OK;
}

static enum sam3_error download(struct sam3_hip_backend *hb, struct s3h_res *e)
{
	enum sam3_error err = s3h_hip(hipMemcpyAsync((void *)e->host, e->dev, e->nbytes,
						     hipMemcpyDeviceToHost, hb->stream),
				      "graph_eval: download");
	if (err == SAM3_OK) {
		e->host_valid = 1;
		hb->stats.downloads++;
	}
	return err;
}

/* ------------------------------------------------------------------ */
/* Graph analysis: how many inputs reference each tensor header.        */
/* ------------------------------------------------------------------ */
struct use_map {
	const struct sam3_tensor **key;
	int *count;
	size_t mask;
};

static size_t ptr_hash(const void *p)
{
	uint64_t x = (uint64_t)(uintptr_t)p;
	x ^= x >> 33;
	x *= 0xff51afd7ed558ccdULL;
	x ^= x >> 33;
	return (size_t)x;
}

static int *use_slot(struct use_map *m, const struct sam3_tensor *t)
{
	size_t i = ptr_hash(t) & m->mask;
	while (m->key[i] && m->key[i] != t)
		i = (i + 1) & m->mask;
	m->key[i] = t;
	return &m->count[i];
}

static int uses_of(struct use_map *m, const struct sam3_tensor *t)
{
	size_t i = ptr_hash(t) & m->mask;
	while (m->key[i]) {
		if (m->key[i] == t)
			return m->count[i];
		i = (i + 1) & m->mask;
	}
	return 0;
}

static enum sam3_error build_uses(const struct sam3_graph *g, struct use_map *m)
{
	size_t want = 16;
	while (want < (size_t)g->n_nodes * 2 * (SAM3_NODE_MAX_INPUTS + 1))
		want <<= 1;
	m->key = calloc(want, sizeof(*m->key));
	m->count = calloc(want, sizeof(*m->count));
	m->mask = want - 1;
	if (!m->key || !m->count) {
		free(m->key);
		free(m->count);
		s3h_error("graph_eval: out of host memory");
		return SAM3_ENOMEM;
	}
	for (int i = 0; i < g->n_nodes; i++) {
		const struct sam3_node *n = &g->nodes[i];
		for (int j = 0; j < n->n_inputs && j < SAM3_NODE_MAX_INPUTS; j++)
			if (n->inputs[j])
				(*use_slot(m, n->inputs[j]))++;
	}
	return SAM3_OK;
}

/* ------------------------------------------------------------------ */
/* Node execution                                                       */
/* ------------------------------------------------------------------ */
static int float_dt(int dt)
{
	return dt == SAM3_DTYPE_F32 || dt == SAM3_DTYPE_F16 || dt == SAM3_DTYPE_BF16;
}

/* A 2-D TRANSPOSE whose only consumer is a later MATMUL's B operand. */
static int transpose_folds(const struct sam3_graph *g, int i, struct use_map *uses)
{
	const struct sam3_node *n = &g->nodes[i];
	if (n->n_inputs < 1 || !n->inputs[0] || !n->output || n->inputs[0]->n_dims != 2 ||
	    !s3h_transpose_is_swap(n) || uses_of(uses, n->output) != 1)
		return 0;
	for (int j = i + 1; j < g->n_nodes; j++) {
		const struct sam3_node *m = &g->nodes[j];
		for (int k = 0; k < m->n_inputs && k < SAM3_NODE_MAX_INPUTS; k++) {
			if (m->inputs[k] != n->output)
				continue;
			return m->op == SAM3_OP_MATMUL && k == 1 && m->n_inputs >= 2 &&
			       m->inputs[0] && (m->inputs[0]->dtype == n->inputs[0]->dtype ||
						n->inputs[0]->dtype == SAM3_DTYPE_Q8_0);
		}
	}
	return 0;
}

static const struct sam3_tensor *folded_source(const struct sam3_graph *g, int upto,
					       const unsigned char *folded,
					       const struct sam3_tensor *t)
{
	for (int j = upto - 1; j >= 0; j--)
		if (folded[j] && g->nodes[j].output == t)
			return g->nodes[j].inputs[0];
	return NULL;
}

static int consumer_operand_form(struct sam3_hip_backend *hb, const struct sam3_graph *g, int i,
				 int j, const struct sam3_tensor *t, int row_len,
				 struct use_map *uses, int *k_out);
static int next_reader(const struct sam3_graph *g, int j, const struct sam3_tensor *t);
static int dims_are(const struct sam3_tensor *t, int B, int S, int H, int D);

/* gh_multihead_attention_rope's q, k and v preparation
 * (graph_helpers.c:721-882): SLICE of the fused qkv output's columns ->
 * RESHAPE [B, S, H, D] -> (ROPE -> RESHAPE ...) -> TRANSPOSE (0, 2, 1, 3).
 * Every tensor in between is used once, so the chain runs as one kernel
 * from the qkv rows to the head-split operand (s3k_rope_split3, which
 * takes the q, k and v chains of one qkv output in one launch), or is
 * stored that way by the qkv GEMM's epilogue (qkv_epilogue_chains). */
struct qkv_chain {
	int n, idx[8];
	const struct sam3_tensor *src, *out, *cos_t, *sin_t;
	long long col0, pitch;
	int B, S, H, D;
};
static int match_qkv_chain(const struct sam3_graph *g, int i, struct use_map *uses,
			   struct qkv_chain *c);

/* Whether a node in [lo, hi) writes tensor r (its header, or its data). */
static int written_between(const struct sam3_graph *g, int lo, int hi,
			   const struct sam3_tensor *r)
{
	for (int k = lo; k < hi; k++) {
		const struct sam3_tensor *o = g->nodes[k].output;
		if (o && (o == r || (o->data && o->data == r->data)))
			return 1;
	}
	return 0;
}

static int in_chains(const struct qkv_chain *cs, int n, int k)
{
	for (int c = 0; c < n; c++)
		for (int t = 0; t < cs[c].n; t++)
			if (cs[c].idx[t] == k)
				return 1;
	return 0;
}

static int same_data(const struct sam3_tensor *a, const struct sam3_tensor *b)
{
	return a && b && (a == b || (a->data && a->data == b->data));
}

/* The q/k/v chains (match_qkv_chain) that are the only readers of the
 * f32 result `out` [M, N] of the GEMM at node i, whose folded nodes end
 * before node j: chain y takes columns [y*E, (y+1)*E), E = H*D, n*E = N,
 * the RoPE chains share one pair of tables, and storing the chains'
 * outputs at node i changes nothing that another node before them reads
 * or writes (no such node touches an output's buffer or writes a table).
 * Returns the number of chains in cs, 0 when they do not fit. */
static int qkv_epilogue_chains(const struct sam3_graph *g, int i, int j,
			       const struct sam3_tensor *out, int M, int N, struct use_map *uses,
			       const unsigned char *done, struct qkv_chain *cs)
{
	const struct s3h_settings *set = s3h_settings();
	if (!set->qkv_fold || !set->qkv_chain)
		return 0;
	const int nu = uses_of(uses, out);
	if (nu < 1 || nu > 3)
		return 0;
	const struct sam3_tensor *ct = NULL, *st = NULL;
	int n = 0, k = j - 1, last = j - 1;
	while (n < nu) {
		k = next_reader(g, k + 1, out);
		if (k < 0 || done[k] || !match_qkv_chain(g, k, uses, &cs[n]) || cs[n].src != out)
			return 0;
		const struct qkv_chain *c = &cs[n];
		if (c->pitch != N || (long long)c->B * c->S != M ||
		    c->col0 != (long long)n * c->H * c->D ||
		    (n && (c->S != cs[0].S || c->H != cs[0].H || c->D != cs[0].D)))
			return 0;
		if (c->cos_t) {
			if (ct && (c->cos_t != ct || c->sin_t != st))
				return 0;
			ct = c->cos_t;
			st = c->sin_t;
		}
		for (int t = 0; t < c->n; t++)
			last = c->idx[t] > last ? c->idx[t] : last;
		n++;
	}
	if ((long long)n * cs[0].H * cs[0].D != N)
		return 0;
	for (int m = i + 1; m <= last; m++) {
		if (m < j || in_chains(cs, n, m))
			continue;
		const struct sam3_node *o = &g->nodes[m];
		if (ct && (same_data(o->output, ct) || same_data(o->output, st)))
			return 0;
		for (int c = 0; c < n; c++) {
			if (same_data(o->output, cs[c].out))
				return 0;
			for (int q = 0; q < o->n_inputs && q < SAM3_NODE_MAX_INPUTS; q++)
				if (same_data(o->inputs[q], cs[c].out))
					return 0;
		}
	}
	return n;
}

/* MATMUL at node i, plus the ADD(bias)/GELU nodes folded into it.
 * Returns the number of nodes consumed in *used. */
static enum sam3_error run_matmul(struct sam3_hip_backend *hb, const struct sam3_graph *g,
				  int i, const unsigned char *folded, unsigned char *done,
				  struct use_map *uses, int *used)
{
	const struct sam3_node *n = &g->nodes[i];
	if (n->n_inputs < 2 || !n->inputs[0] || !n->inputs[1] || !n->output) {
		s3h_error("matmul: NULL tensor");
		return SAM3_EINVAL;
	}
	const struct sam3_tensor *a = n->inputs[0], *b = n->inputs[1];
	const struct sam3_tensor *w = folded_source(g, i, folded, b);
	const int nt = w != NULL;
	const struct sam3_tensor *bsrc = nt ? w : b;
	int a_dt = a->dtype, b_dt = bsrc->dtype;

	/* the same routing as cpu_dispatch_node (cpu_dispatch.c:621-655) */
	if (b_dt == SAM3_DTYPE_Q8_0 ? a_dt != SAM3_DTYPE_F32 : a_dt != b_dt) {
		s3h_error("graph_eval: matmul dtype mismatch a=%d b=%d", a_dt, b_dt);
		return SAM3_EDTYPE;
	}
	if (!float_dt(a_dt)) {
		s3h_error("graph_eval: no matmul kernel for dtype %d", a_dt);
		return SAM3_EDTYPE;
	}
	int M, K, N;
	M = a->n_dims >= 2 ? a->dims[a->n_dims - 2] : 1;
	K = a->n_dims >= 1 ? a->dims[a->n_dims - 1] : 0;
	int kb;
	if (nt) { /* w is [N,K] */
		N = w->dims[0];
		kb = w->dims[1];
	} else {
		kb = b->n_dims >= 2 ? b->dims[b->n_dims - 2] : b->dims[0];
		N = b->n_dims >= 2 ? b->dims[b->n_dims - 1] : 1;
	}
	if (a->n_dims < 1 || kb != K) {
		s3h_error("matmul: K mismatch %d != %d", K, kb);
		return SAM3_EINVAL;
	}
	if (s3h_nelems(n->output) != (long long)M * N) {
		s3h_error("matmul: output size mismatch");
		return SAM3_EINVAL;
	}
	const int c_dt = b_dt == SAM3_DTYPE_Q8_0 ? SAM3_DTYPE_F32 : a_dt;

	/* epilogue folding */
	int flags = nt ? SAM3_HIP_B_NT : 0;
	const struct sam3_tensor *out = n->output, *bias = NULL;
	int j = i + 1;
	if (j < g->n_nodes && g->nodes[j].op == SAM3_OP_ADD && g->nodes[j].n_inputs == 2 &&
	    g->nodes[j].inputs[0] == out && g->nodes[j].inputs[1] &&
	    g->nodes[j].inputs[1] != out && uses_of(uses, out) == 1 &&
	    (int)g->nodes[j].inputs[1]->dtype == c_dt && s3h_nelems(g->nodes[j].inputs[1]) == N &&
	    g->nodes[j].output && s3h_nelems(g->nodes[j].output) == (long long)M * N) {
		bias = g->nodes[j].inputs[1];
		out = g->nodes[j].output;
		flags |= SAM3_HIP_BIAS;
		j++;
	}
	if (j < g->n_nodes && g->nodes[j].op == SAM3_OP_GELU && g->nodes[j].n_inputs >= 1 &&
	    g->nodes[j].inputs[0] == out && uses_of(uses, out) == 1 && g->nodes[j].output &&
	    s3h_nelems(g->nodes[j].output) == (long long)M * N) {
		out = g->nodes[j].output;
		flags |= SAM3_HIP_GELU;
		j++;
	}

	void *da, *db, *dc, *dbias = NULL, *dres = NULL;
	const struct s3h_res *ae = res_find(hb, a->data);
	const int a_fmt = ae ? ae->fmt : S3H_A_PLAIN;
	struct s3h_ln_in ln_a = {NULL, NULL, NULL};
	struct s3h_att1_in att_a;
	enum sam3_error err = dev_in(hb, a, &da);
	if (err == SAM3_OK && a_fmt == S3H_A_LN) {
		/* A is a LayerNorm's output that did not run: the GEMM reads
		 * the LN's input and normalizes it (ln_gemv_form) */
		ln_a.x = ae->ln[0];
		ln_a.gamma = ae->ln[1];
		ln_a.beta = ae->ln[2];
		da = &ln_a;
	} else if (err == SAM3_OK && a_fmt == S3H_A_ATT1) {
		/* A is a one-key attention's merged output that did not run:
		 * the GEMV forms it from q, k and v (sdpa_gemv_form) */
		att_a = ae->att;
		da = &att_a;
	}
	if (err == SAM3_OK)
		err = dev_in(hb, bsrc, &db);
	if (err == SAM3_OK && bias)
		err = dev_in(hb, bias, &dbias);
	if (err != SAM3_OK)
		return err;
	/* gh_window_unpartition (graph_helpers.c:480-509) right after the
	 * GEMM: RESHAPE... -> TRANSPOSE (0,2,1,3) of [d0, d1, d2, g*N] ->
	 * RESHAPE..., every tensor used once, optionally followed by the
	 * residual ADD: a permutation of whole C rows, done by the epilogue's
	 * row map (and the ADD with it); the chain's nodes are marked done */
	int row_map[3] = {0, 0, 0}, chain[10], n_chain = 0;
	if (c_dt == SAM3_DTYPE_F32 && s3h_settings()->unpartition_fold &&
	    s3h_matmul_out_ok(a_fmt, a_dt, da, b_dt, db, M, N, K, flags, S3H_A_PLAIN)) {
		const struct sam3_tensor *t = out;
		int k = j - 1, ok = 0;
		for (;;) {
			if (uses_of(uses, t) != 1 || n_chain >= 8 || (k = next_reader(g, k + 1, t)) < 0)
				break;
			const struct sam3_node *m = &g->nodes[k];
			if (m->inputs[0] != t || !m->output || done[k])
				break;
			if (m->op == SAM3_OP_RESHAPE && s3h_nelems(m->output) == (long long)M * N) {
				chain[n_chain++] = k;
				t = m->output;
			} else if (!ok && m->op == SAM3_OP_TRANSPOSE && t->n_dims == 4 &&
				   m->params[0] == 0 && m->params[1] == 2 && m->params[2] == 1 &&
				   m->params[3] == 3 && m->output->dtype == SAM3_DTYPE_F32 &&
				   t->dims[3] % N == 0 && (long long)t->dims[0] * t->dims[1] * t->dims[2] *
				   t->dims[3] == (long long)M * N) {
				row_map[0] = t->dims[3] / N;
				row_map[1] = t->dims[1];
				row_map[2] = t->dims[2];
				chain[n_chain++] = k;
				t = m->output;
				ok = 1;
			} else {
				break;
			}
		}
		/* the residual ADD of the unpartitioned result completes the fold
		 * (its output, unlike the views before it, has its own buffer) */
		int fold = 0;
		if (ok) {
			const int ka = uses_of(uses, t) == 1 ? next_reader(g, chain[n_chain - 1] + 1, t) : -1;
			const struct sam3_node *ad = ka >= 0 ? &g->nodes[ka] : NULL;
			const struct sam3_tensor *r = NULL;
			if (ad && ad->op == SAM3_OP_ADD && ad->n_inputs == 2 && ad->output && !done[ka])
				r = ad->inputs[0] == t ? ad->inputs[1] : ad->inputs[1] == t ? ad->inputs[0] : NULL;
			/* the epilogue reads r when the GEMM runs, so no node between
			 * the GEMM and the ADD may write it */
			if (r && r != t && r->data && r->dtype == SAM3_DTYPE_F32 &&
			    ad->output->dtype == SAM3_DTYPE_F32 && s3h_nelems(r) == (long long)M * N &&
			    s3h_nelems(ad->output) == (long long)M * N && r->data != ad->output->data &&
			    !written_between(g, i + 1, ka, r) && dev_in(hb, r, &dres) == SAM3_OK) {
				chain[n_chain++] = ka;
				out = ad->output;
				fold = 1;
			} else {
				dres = NULL;
			}
		}
		if (!fold) {
			n_chain = 0;
			row_map[0] = 0;
		}
	}
	/* a residual ADD of an f32 [M, N] tensor computed earlier (the
	 * block's x + attention / + MLP), folded last into the epilogue */
	if (!row_map[0] && c_dt == SAM3_DTYPE_F32 && s3h_settings()->residual_fold && j < g->n_nodes &&
	    g->nodes[j].op == SAM3_OP_ADD && g->nodes[j].n_inputs == 2 && g->nodes[j].output &&
	    uses_of(uses, out) == 1 &&
	    s3h_nelems(g->nodes[j].output) == (long long)M * N) {
		const struct sam3_node *ad = &g->nodes[j];
		const struct sam3_tensor *r = ad->inputs[0] == out ? ad->inputs[1]
					      : ad->inputs[1] == out ? ad->inputs[0] : NULL;
		if (r && r != out && r->data && r->dtype == SAM3_DTYPE_F32 &&
		    ad->output->dtype == SAM3_DTYPE_F32 && s3h_nelems(r) == (long long)M * N &&
		    r->data != ad->output->data &&
		    s3h_matmul_res_ok(a_fmt, a_dt, da, b_dt, db, M, N, K, flags) &&
		    !written_between(g, i + 1, j, r) && dev_in(hb, r, &dres) == SAM3_OK) {
			out = ad->output;
			j++;
		} else {
			dres = NULL;
		}
	}
	/* an f32 result read only by the next GEMM, which converts its A
	 * first: written in that form by this GEMM's epilogue */
	int o_fmt = S3H_A_PLAIN;
	if (!row_map[0] && c_dt == SAM3_DTYPE_F32 && s3h_settings()->gemm_operand) {
		o_fmt = consumer_operand_form(hb, g, i, j, out, N, uses, NULL);
		if (o_fmt != S3H_A_PLAIN &&
		    !s3h_matmul_out_ok(a_fmt, a_dt, da, b_dt, db, M, N, K, flags, o_fmt))
			o_fmt = S3H_A_PLAIN;
	}
	/* an f32 result read only by the q/k/v chains of attention: stored
	 * by the epilogue as their head-split outputs (RoPE applied) */
	struct qkv_chain qcs[3];
	int n_qkv = 0;
	struct s3h_qkv qkv;
	memset(&qkv, 0, sizeof(qkv));
	if (o_fmt == S3H_A_PLAIN && !dres && !row_map[0] && c_dt == SAM3_DTYPE_F32 &&
	    (n_qkv = qkv_epilogue_chains(g, i, j, out, M, N, uses, done, qcs)) > 0) {
		static const float al[4] __attribute__((aligned(16)));
		qkv.S = qcs[0].S;
		qkv.H = qcs[0].H;
		qkv.D = qcs[0].D;
		for (int y = 0; y < n_qkv; y++) {
			qkv.out[y] = (float *)al;
			qkv.rope |= (qcs[y].cos_t != NULL) << y;
			if (qcs[y].cos_t) {
				qkv.cos_t = al;
				qkv.sin_t = al;
			}
		}
		if (!s3h_matmul_qkv_ok(a_fmt, a_dt, da, b_dt, db, M, N, K, flags, &qkv) ||
		    (bias && ((uintptr_t)dbias & 15u)))
			n_qkv = 0;
	}
	if (n_qkv) {
		const struct sam3_tensor *ct = NULL, *st = NULL;
		for (int y = 0; y < n_qkv && err == SAM3_OK; y++) {
			void *dy = NULL;
			err = dev_out(hb, qcs[y].out, &dy);
			qkv.out[y] = (float *)dy;
			if (qcs[y].cos_t) {
				ct = qcs[y].cos_t;
				st = qcs[y].sin_t;
			}
		}
		void *dct = NULL, *dst = NULL;
		if (err == SAM3_OK && ct)
			err = dev_in(hb, ct, &dct);
		if (err == SAM3_OK && st)
			err = dev_in(hb, st, &dst);
		qkv.cos_t = (const float *)dct;
		qkv.sin_t = (const float *)dst;
		if (err == SAM3_OK)
			err = s3h_matmul_qkv(a_fmt, a_dt, da, b_dt, db, M, N, K, dbias, flags, &qkv,
					     hb->stream);
		if (err == SAM3_OK)
			for (int y = 0; y < n_qkv; y++) {
				for (int t = 0; t < qcs[y].n; t++)
					done[qcs[y].idx[t]] = 1;
				n_chain += qcs[y].n;
			}
	} else if (o_fmt != S3H_A_PLAIN) {
		/* an f16 operand carries its row tags (two words per row) after
		 * the data: zeroed when the allocation is new to this form, then
		 * stamped with each eval's own tag */
		const size_t dbytes = ((size_t)M * N * (o_fmt == S3H_A_PLANES ? 6 : 2) + 15) & ~(size_t)15;
		const int f16 = o_fmt == S3H_A_F16;
		int same = 0;
		unsigned *rowf = NULL;
		err = dev_out_fmt(hb, out, dbytes + (f16 ? (size_t)M * 8 : 0), o_fmt, &dc, &same);
		if (err == SAM3_OK && f16) {
			rowf = (unsigned *)((char *)dc + dbytes);
			if (!same)
				err = s3h_hip(hipMemsetAsync(rowf, 0, (size_t)M * 8, hb->stream),
					      "graph_eval: row tags");
			if (err == SAM3_OK && hb->n_rowf == 32)
				err = rowf_flush(hb);
		}
		if (err == SAM3_OK)
			err = s3h_matmul_fmt_to(a_fmt, o_fmt, a_dt, da, b_dt, db, dc, M, N, K, dbias,
						dres, NULL, flags, hb->ovf, hb->ovf_tag, rowf,
						hb->stream);
		if (err == SAM3_OK) {
			hb->stats.operand_writes++;
			hb->f16_writes += f16;
			if (f16) {
				hb->rowf[hb->n_rowf] = rowf;
				hb->rowf_rows[hb->n_rowf++] = M;
			}
		}
	} else if (dres || row_map[0]) {
		err = dev_out(hb, out, &dc);
		if (err == SAM3_OK)
			err = s3h_matmul_fmt_to(a_fmt, S3H_A_PLAIN, a_dt, da, b_dt, db, dc, M, N, K,
						dbias, dres, row_map[0] ? row_map : NULL, flags, NULL,
						0, NULL, hb->stream);
		if (err == SAM3_OK)
			for (int k = 0; k < n_chain; k++)
				done[chain[k]] = 1;
	} else {
		err = dev_out(hb, out, &dc);
		if (err != SAM3_OK)
			return err;
		err = a_fmt ? s3h_matmul_fmt(a_fmt, a_dt, da, b_dt, db, c_dt, dc, M, N, K, dbias,
					     flags, hb->stream)
			    : sam3_hip_matmul(a_dt, da, b_dt, db, c_dt, dc, M, N, K, dbias, flags,
					      hb->stream);
	}
	if (err == SAM3_OK) {
		hb->stats.gpu_nodes++;
		hb->stats.fused_nodes += j - i - 1 + n_chain;
		*used = j - i;
	}
	return err;
}

/* The MATMUL that reads tensor t, produced by node i (or by the chain of
 * nodes folded into it, the last of them before node j), as its A: t
 * used once, through RESHAPE views only. Fills r (the MATMUL's index, its
 * A view, the weight tensor it uses - the source of a folded TRANSPOSE
 * when its B is one, then nt = 1 - and the GEMM's M, N, K). */
struct gemm_reader {
	int j, nt, M, N, K;
	const struct sam3_tensor *a, *w;
};
static int find_gemm_reader(const struct sam3_graph *g, int i, int j, const struct sam3_tensor *t,
			    struct use_map *uses, struct gemm_reader *r)
{
	for (;;) {
		if (uses_of(uses, t) != 1)
			return 0;
		while (j < g->n_nodes) {
			const struct sam3_node *m = &g->nodes[j];
			int hit = 0;
			for (int k = 0; k < m->n_inputs && k < SAM3_NODE_MAX_INPUTS; k++)
				hit |= m->inputs[k] == t;
			if (hit)
				break;
			j++;
		}
		if (j >= g->n_nodes)
			return 0;
		if (g->nodes[j].op != SAM3_OP_RESHAPE || g->nodes[j].inputs[0] != t)
			break;
		t = g->nodes[j].output;
		j++;
	}
	const struct sam3_node *mm = &g->nodes[j];
	if (mm->op != SAM3_OP_MATMUL || mm->n_inputs < 2 || mm->inputs[0] != t || !mm->inputs[1] ||
	    !mm->output)
		return 0;
	const struct sam3_tensor *b = mm->inputs[1], *w = NULL;
	for (int k = i + 1; k < j && !w; k++)
		if (g->nodes[k].op == SAM3_OP_TRANSPOSE && g->nodes[k].output == b &&
		    transpose_folds(g, k, uses))
			w = g->nodes[k].inputs[0];
	const struct sam3_tensor *bsrc = w ? w : b;
	if (!bsrc->data || t->n_dims < 1)
		return 0;
	const int M = t->n_dims >= 2 ? t->dims[t->n_dims - 2] : 1, K = t->dims[t->n_dims - 1];
	int N, kb;
	if (w) {
		N = w->dims[0];
		kb = w->dims[1];
	} else {
		kb = b->n_dims >= 2 ? b->dims[b->n_dims - 2] : b->dims[0];
		N = b->n_dims >= 2 ? b->dims[b->n_dims - 1] : 1;
	}
	if (kb != K || s3h_nelems(t) != (long long)M * K)
		return 0;
	r->j = j;
	r->a = t;
	r->w = bsrc;
	r->nt = w != NULL;
	r->M = M;
	r->N = N;
	r->K = K;
	return 1;
}

/* The GEMM operand form in which tensor t, produced by node i (or by the
 * chain of nodes folded into it, the last of them before node j), can be
 * written: t must be used once, through RESHAPE views only, as the A of a
 * MATMUL that converts A before its GEMM (s3h_matmul_a_format), with
 * rows of row_len values (the producer's row length). The consumer's
 * weight is resolved (and uploaded) here to decide with its device
 * address. */
static int consumer_operand_form(struct sam3_hip_backend *hb, const struct sam3_graph *g, int i,
				 int j, const struct sam3_tensor *t, int row_len,
				 struct use_map *uses, int *k_out)
{
	struct gemm_reader r;
	if (!find_gemm_reader(g, i, j, t, uses, &r) || (row_len > 0 && r.K != row_len))
		return S3H_A_PLAIN;
	if (k_out)
		*k_out = r.K;
	void *db = NULL;
	if (dev_in(hb, r.w, &db) != SAM3_OK)
		return S3H_A_PLAIN;
	static const char aligned_a[16] __attribute__((aligned(16)));
	const int f = s3h_matmul_a_format(SAM3_DTYPE_F32, aligned_a, r.w->dtype, db, SAM3_DTYPE_F32,
					  r.M, r.N, r.K, r.nt ? SAM3_HIP_B_NT : 0);
	return f == S3H_A_F16 && hb->no_f16_ops ? S3H_A_PLAIN : f;
}

/* The form an f32 LAYERNORM at node i writes: its consumer's operand. */
static int ln_operand_form(struct sam3_hip_backend *hb, const struct sam3_graph *g, int i,
			   struct use_map *uses)
{
	const struct sam3_node *n = &g->nodes[i];
	if (n->inputs[0]->dtype != SAM3_DTYPE_F32 || !s3h_layernorm_ok(n))
		return S3H_A_PLAIN;
	return consumer_operand_form(hb, g, i, i + 1, n->output,
				     n->inputs[0]->dims[n->inputs[0]->n_dims - 1], uses, NULL);
}

/* Whether a node after node i writes tensor r's data. */
static int written_after(const struct sam3_graph *g, int i, const struct sam3_tensor *r)
{
	if (!r)
		return 0;
	for (int k = i + 1; k < g->n_nodes; k++) {
		const struct sam3_tensor *o = g->nodes[k].output;
		if (o && (o == r || (o->data && o->data == r->data)))
			return 1;
	}
	return 0;
}

/* An f32 LAYERNORM at node i whose output only a Q8_0 GEMM on the
 * streaming skinny kernel reads (through RESHAPE views): the LN does not
 * run; the GEMM normalizes its rows as it reads the LN's input
 * (S3H_A_LN, the same arithmetic, so the same bits). No later node may
 * write the LN's input, gamma or beta, which the GEMM reads when it runs.
 * Fills ln with their device addresses. */
static int ln_gemv_form(struct sam3_hip_backend *hb, const struct sam3_graph *g, int i,
			struct use_map *uses, struct s3h_ln_in *ln)
{
	const struct sam3_node *n = &g->nodes[i];
	if (!s3h_settings()->ln_gemv_fold || n->inputs[0]->dtype != SAM3_DTYPE_F32 ||
	    !s3h_layernorm_ok(n))
		return 0;
	const struct sam3_tensor *x = n->inputs[0];
	const struct sam3_tensor *gm = n->n_inputs > 1 ? n->inputs[1] : NULL;
	const struct sam3_tensor *bt = n->n_inputs > 2 ? n->inputs[2] : NULL;
	struct gemm_reader r;
	if (!find_gemm_reader(g, i, i + 1, n->output, uses, &r) || !r.nt ||
	    r.w->dtype != SAM3_DTYPE_Q8_0 || r.K != x->dims[x->n_dims - 1] ||
	    (long long)r.M * r.K != s3h_nelems(x) || !x->data || written_after(g, i, x) ||
	    written_after(g, i, gm) || written_after(g, i, bt))
		return 0;
	const struct s3h_res *xe = res_find(hb, x->data);
	if (xe && xe->fmt)
		return 0;
	void *dx = NULL, *dg = NULL, *dbt = NULL, *dw = NULL;
	if (dev_in(hb, x, &dx) != SAM3_OK || (gm && dev_in(hb, gm, &dg) != SAM3_OK) ||
	    (bt && dev_in(hb, bt, &dbt) != SAM3_OK) || dev_in(hb, r.w, &dw) != SAM3_OK)
		return 0;
	ln->x = dx;
	ln->gamma = dg;
	ln->beta = dbt;
	return s3h_matmul_ln_ok(r.w->dtype, dw, r.M, r.N, r.K, SAM3_HIP_B_NT, ln);
}

/* LAYERNORM left to its consuming GEMM: the output's residency entry
 * holds the form S3H_A_LN and the device addresses in ln. */
static enum sam3_error run_layernorm_gemv(struct sam3_hip_backend *hb, const struct sam3_node *n,
					  const struct s3h_ln_in *ln)
{
	void *dy = NULL;
	enum sam3_error err = dev_out_fmt(hb, n->output, 256, S3H_A_LN, &dy, NULL);
	if (err != SAM3_OK)
		return err;
	struct s3h_res *e = res_find(hb, n->output->data);
	if (!e) {
		s3h_error("graph_eval: LayerNorm output not resident");
		return SAM3_EBACKEND;
	}
	e->ln[0] = ln->x;
	e->ln[1] = ln->gamma;
	e->ln[2] = ln->beta;
	hb->stats.fused_nodes++;
	return SAM3_OK;
}

/* gh_sdpa (graph_helpers.c:688-717) of one query over one key per head
 * (the text encoder at one token, text_encoder.c:588-652), f32, batch 1,
 * whose head-merged output (TRANSPOSE (0,2,1,3), then RESHAPE views) only
 * a Q8_0 GEMM of one row reads: the attention does not run. The f32 GEMV
 * forms its output from q, k and v (S3H_A_ATT1) with the steps of the
 * kernel that would have run (attn_generic), so the bits are the same.
 * No later node may write q, k, v or the mask, which the GEMV reads when
 * it runs. Returns the transpose's node index (or -1) and fills at with
 * device addresses. */
static int sdpa_gemv_form(struct sam3_hip_backend *hb, const struct sam3_graph *g, int i,
			  struct use_map *uses, const unsigned char *done, struct s3h_att1_in *at)
{
	const struct sam3_node *n = &g->nodes[i];
	if (!s3h_settings()->att_gemv_fold || !s3h_settings()->sdpa_merge || !s3h_sdpa_node_ok(n))
		return -1;
	const struct sam3_tensor *q = n->inputs[0], *k = n->inputs[1], *v = n->inputs[2];
	const struct sam3_tensor *mk = n->n_inputs > 3 ? n->inputs[3] : NULL, *o = n->output;
	const int D = n->params[0];
	if (q->dtype != SAM3_DTYPE_F32 || q->n_dims != 4 || q->dims[0] != 1 || q->dims[2] != 1)
		return -1;
	const int H = q->dims[1];
	if (!dims_are(q, 1, H, 1, D) || !dims_are(k, 1, H, 1, D) || !dims_are(v, 1, H, 1, D) ||
	    !dims_are(o, 1, H, 1, D) || uses_of(uses, o) != 1 || (mk && s3h_nelems(mk) != 1))
		return -1;
	const int j = next_reader(g, i + 1, o);
	if (j < 0 || done[j])
		return -1;
	const struct sam3_node *t = &g->nodes[j];
	if (t->op != SAM3_OP_TRANSPOSE || t->n_inputs < 1 || t->inputs[0] != o || !t->output ||
	    t->params[0] != 0 || t->params[1] != 2 || t->params[2] != 1 || t->params[3] != 3 ||
	    t->output->dtype != SAM3_DTYPE_F32 || !dims_are(t->output, 1, 1, H, D))
		return -1;
	struct gemm_reader r;
	if (!find_gemm_reader(g, j, j + 1, t->output, uses, &r) || !r.nt ||
	    r.w->dtype != SAM3_DTYPE_Q8_0 || r.M != 1 || r.K != H * D || written_after(g, i, q) ||
	    written_after(g, i, k) || written_after(g, i, v) || written_after(g, i, mk))
		return -1;
	for (int m = i + 1; m < j; m++) {
		const struct sam3_node *x = &g->nodes[m];
		if (same_data(x->output, t->output))
			return -1;
	}
	void *dq = NULL, *dk = NULL, *dv = NULL, *dm = NULL, *dw = NULL;
	if (dev_in(hb, q, &dq) != SAM3_OK || dev_in(hb, k, &dk) != SAM3_OK ||
	    dev_in(hb, v, &dv) != SAM3_OK || (mk && dev_in(hb, mk, &dm) != SAM3_OK) ||
	    dev_in(hb, r.w, &dw) != SAM3_OK)
		return -1;
	/* the kernel the unfolded node would run, writing aligned rows */
	static const float al[4] __attribute__((aligned(16)));
	if (s3k_attn_heads_path(S3K_F32, dq, dk, dv, (void *)al, H, 1, 1, D, H, 0) !=
	    S3K_ATTN_GENERIC)
		return -1;
	at->q = dq;
	at->k = dk;
	at->v = dv;
	at->mask = dm;
	at->scale = 1.0f / sqrtf((float)D);
	at->D = D;
	return s3h_matmul_att1_ok(r.w->dtype, dw, r.M, r.N, r.K, SAM3_HIP_B_NT, at) ? j : -1;
}

/* SDPA (and its head-merge TRANSPOSE t) left to the consuming GEMV: t's
 * output holds the form S3H_A_ATT1 and the device addresses in at. */
static enum sam3_error run_sdpa_gemv(struct sam3_hip_backend *hb, const struct sam3_node *t,
				     const struct s3h_att1_in *at)
{
	void *dy = NULL;
	enum sam3_error err = dev_out_fmt(hb, t->output, 256, S3H_A_ATT1, &dy, NULL);
	if (err != SAM3_OK)
		return err;
	struct s3h_res *e = res_find(hb, t->output->data);
	if (!e) {
		s3h_error("graph_eval: attention output not resident");
		return SAM3_EBACKEND;
	}
	e->att = *at;
	hb->stats.fused_nodes += 2;
	return SAM3_OK;
}

/* The form an f32 TRANSPOSE at node i that keeps its last axis writes:
 * its consumer's operand, read as rows of *K values. */
static int permute_operand_form(struct sam3_hip_backend *hb, const struct sam3_graph *g, int i,
				struct use_map *uses, int *K)
{
	const struct sam3_node *n = &g->nodes[i];
	if (n->n_inputs < 1 || !n->inputs[0] || !n->output || n->inputs[0]->dtype != SAM3_DTYPE_F32 ||
	    !s3h_transpose_to_ok(n, 4))
		return S3H_A_PLAIN;
	int k = 0;
	const int f = consumer_operand_form(hb, g, i, i + 1, n->output, 0, uses, &k);
	if (f == S3H_A_PLAIN || !s3h_transpose_to_ok(n, k))
		return S3H_A_PLAIN;
	*K = k;
	return f;
}

/* gh_multihead_attention_rope's q, k and v preparation
 * (graph_helpers.c:721-882): match_qkv_chain below. */

static int next_reader(const struct sam3_graph *g, int j, const struct sam3_tensor *t)
{
	for (; j < g->n_nodes; j++) {
		const struct sam3_node *m = &g->nodes[j];
		for (int k = 0; k < m->n_inputs && k < SAM3_NODE_MAX_INPUTS; k++)
			if (m->inputs[k] == t)
				return j;
	}
	return -1;
}

static int dims_are(const struct sam3_tensor *t, int B, int S, int H, int D)
{
	return t && t->n_dims == 4 && t->dims[0] == B && t->dims[1] == S && t->dims[2] == H &&
	       t->dims[3] == D;
}

static int match_qkv_chain(const struct sam3_graph *g, int i, struct use_map *uses,
			   struct qkv_chain *c)
{
	const struct sam3_node *n = &g->nodes[i];
	if (n->op != SAM3_OP_SLICE || n->n_inputs < 1 || !n->inputs[0] || !n->output ||
	    !s3h_slice_ok(n))
		return 0;
	const struct sam3_tensor *x = n->inputs[0];
	const int c0 = n->params[1], c1 = n->params[2];
	if (x->dtype != SAM3_DTYPE_F32 || x->n_dims != 2 || n->params[0] != 1 || c0 % 4 ||
	    x->dims[1] % 4 || c1 <= c0 || c1 > x->dims[1])
		return 0;
	c->n = 0;
	c->idx[c->n++] = i;
	const struct sam3_tensor *t = n->output;
	int j = i;
	if (uses_of(uses, t) != 1 || (j = next_reader(g, j + 1, t)) < 0 ||
	    g->nodes[j].op != SAM3_OP_RESHAPE || !g->nodes[j].output)
		return 0;
	c->idx[c->n++] = j;
	t = g->nodes[j].output;
	if (t->n_dims != 4)
		return 0;
	const int B = t->dims[0], S = t->dims[1], H = t->dims[2], D = t->dims[3];
	if ((long long)B * S != x->dims[0] || (long long)H * D != c1 - c0 || D % 4)
		return 0;
	c->cos_t = c->sin_t = NULL;
	for (;;) {
		if (uses_of(uses, t) != 1 || (j = next_reader(g, j + 1, t)) < 0 || c->n >= 8)
			return 0;
		const struct sam3_node *m = &g->nodes[j];
		if (!m->output || m->inputs[0] != t)
			return 0;
		if (m->op == SAM3_OP_RESHAPE && s3h_nelems(m->output) == (long long)B * S * H * D) {
			c->idx[c->n++] = j;
			t = m->output;
		} else if (m->op == SAM3_OP_ROPE && !c->cos_t && dims_are(t, B, S, H, D) &&
			   s3h_rope_ok(m) && m->output->dtype == SAM3_DTYPE_F32) {
			c->cos_t = m->inputs[1];
			c->sin_t = m->inputs[2];
			c->idx[c->n++] = j;
			t = m->output;
		} else if (m->op == SAM3_OP_TRANSPOSE && dims_are(t, B, S, H, D) && m->params[0] == 0 &&
			   m->params[1] == 2 && m->params[2] == 1 && m->params[3] == 3 &&
			   dims_are(m->output, B, H, S, D) && m->output->dtype == SAM3_DTYPE_F32) {
			c->idx[c->n++] = j;
			c->out = m->output;
			break;
		} else {
			return 0;
		}
	}
	c->src = x;
	c->col0 = c0;
	c->pitch = x->dims[1];
	c->B = B;
	c->S = S;
	c->H = H;
	c->D = D;
	return 1;
}

/* The chain c0 at node c0->idx[0] and the next (up to two) chains that
 * slice the same qkv rows with the same head split (k and v after q), as
 * one launch of s3k_rope_split3. A later chain joins only if no node
 * before it writes the rows or the RoPE tables it reads, and the RoPE
 * chains share one pair of tables. */
static enum sam3_error run_qkv_chains(struct sam3_hip_backend *hb, const struct sam3_graph *g,
				      const struct qkv_chain *c0, struct use_map *uses,
				      unsigned char *done)
{
	struct qkv_chain cs[3];
	int n = 1;
	cs[0] = *c0;
	const struct sam3_tensor *ct = c0->cos_t, *st = c0->sin_t;
	const int i = c0->idx[0];
	for (int j = i + 1; j < g->n_nodes && n < 3; j++) {
		const struct sam3_node *m = &g->nodes[j];
		if (done[j] || m->op != SAM3_OP_SLICE || m->n_inputs < 1 || m->inputs[0] != c0->src)
			continue;
		struct qkv_chain c;
		if (!match_qkv_chain(g, j, uses, &c) || c.B != c0->B || c.S != c0->S || c.H != c0->H ||
		    c.D != c0->D || c.pitch != c0->pitch)
			break;
		if (c.cos_t && ct && (c.cos_t != ct || c.sin_t != st))
			break;
		if (written_between(g, i + 1, j, c0->src) ||
		    (c.cos_t && (written_between(g, i + 1, j, c.cos_t) ||
				 written_between(g, i + 1, j, c.sin_t))))
			break;
		if (c.cos_t) {
			ct = c.cos_t;
			st = c.sin_t;
		}
		cs[n++] = c;
	}
	void *dx = NULL, *dc = NULL, *ds = NULL;
	float *outs[3] = {NULL, NULL, NULL};
	long long cols[3] = {0, 0, 0};
	int rope_mask = 0;
	enum sam3_error err = dev_in(hb, c0->src, &dx);
	if (err == SAM3_OK && ct)
		err = dev_in(hb, ct, &dc);
	if (err == SAM3_OK && st)
		err = dev_in(hb, st, &ds);
	for (int k = 0; k < n && err == SAM3_OK; k++) {
		void *dy = NULL;
		err = dev_out(hb, cs[k].out, &dy);
		outs[k] = (float *)dy;
		cols[k] = cs[k].col0;
		rope_mask |= (cs[k].cos_t != NULL) << k;
	}
	if (err == SAM3_OK)
		err = s3h_hip(s3k_rope_split3((const float *)dx, c0->pitch, cols, (const float *)dc,
					      (const float *)ds, rope_mask, outs, n, c0->B, c0->S,
					      c0->H, c0->D, hb->stream),
			      "attention operands (slice, rope, head split)");
	if (err != SAM3_OK)
		return err;
	int fused = -1;
	for (int k = 0; k < n; k++) {
		for (int t = k ? 0 : 1; t < cs[k].n; t++)
			done[cs[k].idx[t]] = 1;
		fused += cs[k].n;
	}
	hb->stats.gpu_nodes++;
	hb->stats.fused_nodes += fused;
	return SAM3_OK;
}

/* TRANSPOSE written as the operand form fmt of its one consuming GEMM. */
static enum sam3_error run_permute_as(struct sam3_hip_backend *hb, const struct sam3_node *n,
				      int fmt, int K)
{
	void *dx = NULL, *dy = NULL;
	enum sam3_error err = dev_in(hb, n->inputs[0], &dx);
	if (err == SAM3_OK)
		err = dev_out_fmt(hb, n->output,
				  (size_t)s3h_nelems(n->output) * (fmt == S3H_A_PLANES ? 6 : 2), fmt, &dy,
				  NULL);
	if (err == SAM3_OK)
		err = s3h_transpose_to(n, dx, dy, fmt, K, hb->ovf, hb->ovf_tag, hb->stream);
	if (err == SAM3_OK) {
		hb->stats.gpu_nodes++;
		hb->stats.operand_writes++;
		hb->f16_writes += fmt == S3H_A_F16;
	}
	return err;
}

/* An f32 LAYERNORM followed by gh_window_partition (graph_helpers.c:
 * 447-478: RESHAPE -> TRANSPOSE (0,2,1,3) of [d0, d1, d2, g*cols] ->
 * RESHAPE ...) whose result only a GEMM reads, as its A: the LN writes
 * that GEMM's operand with its rows already in partition order (a store
 * row map), under the GEMM's A tensor. Returns the form; rm, the chain's
 * node indices and that tensor are filled in. */
static int ln_partition_form(struct sam3_hip_backend *hb, const struct sam3_graph *g, int i,
			     struct use_map *uses, int rm[3], int *chain, int *n_chain,
			     const struct sam3_tensor **a_out)
{
	const struct sam3_node *n = &g->nodes[i];
	if (n->inputs[0]->dtype != SAM3_DTYPE_F32 || !s3h_layernorm_ok(n))
		return S3H_A_PLAIN;
	const int cols = n->inputs[0]->dims[n->inputs[0]->n_dims - 1];
	const long long tot = s3h_nelems(n->inputs[0]);
	const struct sam3_tensor *t = n->output;
	int k = i, nc = 0, ok = 0;
	for (;;) {
		if (uses_of(uses, t) != 1 || nc >= 8 || (k = next_reader(g, k + 1, t)) < 0)
			break;
		const struct sam3_node *m = &g->nodes[k];
		if (m->inputs[0] != t || !m->output)
			break;
		if (m->op == SAM3_OP_RESHAPE && s3h_nelems(m->output) == tot) {
			chain[nc++] = k;
			t = m->output;
		} else if (!ok && m->op == SAM3_OP_TRANSPOSE && t->n_dims == 4 && m->params[0] == 0 &&
			   m->params[1] == 2 && m->params[2] == 1 && m->params[3] == 3 &&
			   m->output->dtype == SAM3_DTYPE_F32 && t->dims[3] % cols == 0 &&
			   s3h_nelems(t) == tot) {
			rm[0] = t->dims[3] / cols;
			rm[1] = t->dims[1];
			rm[2] = t->dims[2];
			chain[nc++] = k;
			t = m->output;
			ok = 1;
		} else {
			break;
		}
	}
	if (!ok || !t->data)
		return S3H_A_PLAIN;
	const int fmt = consumer_operand_form(hb, g, i, chain[nc - 1] + 1, t, cols, uses, NULL);
	if (fmt == S3H_A_PLAIN)
		return S3H_A_PLAIN;
	*n_chain = nc;
	*a_out = t;
	return fmt;
}

/* LAYERNORM written as that operand, rows in partition order, under t. */
static enum sam3_error run_layernorm_map(struct sam3_hip_backend *hb, const struct sam3_node *n,
					 int fmt, const int rm[3], const struct sam3_tensor *t)
{
	const struct sam3_tensor *x = n->inputs[0];
	const int cols = x->dims[x->n_dims - 1];
	const long long rows = s3h_nelems(x) / cols;
	void *dx = NULL, *dg = NULL, *db = NULL, *dy = NULL;
	enum sam3_error err = dev_in(hb, x, &dx);
	if (err == SAM3_OK && n->n_inputs > 1 && n->inputs[1])
		err = dev_in(hb, n->inputs[1], &dg);
	if (err == SAM3_OK && n->n_inputs > 2 && n->inputs[2])
		err = dev_in(hb, n->inputs[2], &db);
	if (err == SAM3_OK)
		err = dev_out_fmt(hb, t, (size_t)rows * cols * (fmt == S3H_A_PLANES ? 6 : 2), fmt, &dy,
				  NULL);
	if (err == SAM3_OK)
		err = s3h_hip(s3k_layernorm_to_map(fmt == S3H_A_PLANES ? S3K_LN_PLANES : S3K_LN_F16,
						   (const float *)dx, (const float *)dg,
						   (const float *)db, dy, rows, cols, rm[0], rm[1], rm[2],
						   hb->ovf, hb->ovf_tag, hb->stream),
			      "layernorm (GEMM operand, partition order)");
	if (err == SAM3_OK) {
		hb->stats.gpu_nodes++;
		hb->stats.operand_writes++;
		hb->f16_writes += fmt == S3H_A_F16;
	}
	return err;
}

/* LAYERNORM written as the operand form fmt of its one consuming GEMM. */
static enum sam3_error run_layernorm_as(struct sam3_hip_backend *hb, const struct sam3_node *n,
					int fmt)
{
	const struct sam3_tensor *x = n->inputs[0];
	const int cols = x->dims[x->n_dims - 1];
	const long long rows = s3h_nelems(x) / cols;
	void *dx = NULL, *dg = NULL, *db = NULL, *dy = NULL;
	enum sam3_error err = dev_in(hb, x, &dx);
	if (err == SAM3_OK && n->n_inputs > 1 && n->inputs[1])
		err = dev_in(hb, n->inputs[1], &dg);
	if (err == SAM3_OK && n->n_inputs > 2 && n->inputs[2])
		err = dev_in(hb, n->inputs[2], &db);
	if (err == SAM3_OK)
		err = dev_out_fmt(hb, n->output, (size_t)rows * cols * (fmt == S3H_A_PLANES ? 6 : 2),
				  fmt, &dy, NULL);
	if (err == SAM3_OK)
		err = s3h_hip(s3k_layernorm_to(fmt == S3H_A_PLANES ? S3K_LN_PLANES : S3K_LN_F16,
					       (const float *)dx, (const float *)dg,
					       (const float *)db, dy, rows, cols, hb->ovf, hb->ovf_tag,
					       hb->stream),
			      "layernorm (GEMM operand)");
	if (err == SAM3_OK)
		hb->f16_writes += fmt == S3H_A_F16;
	if (err == SAM3_OK) {
		hb->stats.gpu_nodes++;
		hb->stats.operand_writes++;
	}
	return err;
}

/* CONV2D or CONV_TRANSPOSE2D at node i, plus a following BIAS_ADD ([OC],
 * used only there) and GELU folded into the GEMM epilogue when the conv
 * runs as a GEMM. */
static enum sam3_error run_conv(struct sam3_hip_backend *hb, const struct sam3_graph *g, int i,
				struct use_map *uses, int *used)
{
	const int transposed = g->nodes[i].op == SAM3_OP_CONV_TRANSPOSE2D;
	const struct sam3_node *n = &g->nodes[i];
	struct sam3_tensor tx = *n->inputs[0], tw = *n->inputs[1], ty = *n->output;
	struct sam3_node dn = *n;
	enum sam3_error err = dev_in(hb, n->inputs[0], &tx.data);
	if (err == SAM3_OK)
		err = dev_in(hb, n->inputs[1], &tw.data);
	if (err != SAM3_OK)
		return err;
	dn.inputs[0] = &tx;
	dn.inputs[1] = &tw;
	dn.output = &ty;
	/* the kernel choice looks at the device addresses */
	const int path = transposed ? s3h_conv_transpose2d_path(&dn) : s3h_conv2d_path(&dn);
	const struct sam3_tensor *out = n->output, *bias = NULL;
	const long long ny = s3h_nelems(out);
	int flags = 0, j = i + 1;
	if (path != S3H_CONV_DIRECT && j < g->n_nodes && g->nodes[j].op == SAM3_OP_BIAS_ADD &&
	    g->nodes[j].n_inputs == 2 && g->nodes[j].inputs[0] == out && g->nodes[j].inputs[1] &&
	    g->nodes[j].inputs[1] != out && uses_of(uses, out) == 1 &&
	    g->nodes[j].inputs[1]->dtype == out->dtype &&
	    s3h_nelems(g->nodes[j].inputs[1]) == out->dims[3] && g->nodes[j].output &&
	    s3h_nelems(g->nodes[j].output) == ny) {
		bias = g->nodes[j].inputs[1];
		out = g->nodes[j].output;
		flags |= S3K_EPI_BIAS;
		j++;
	}
	if (path != S3H_CONV_DIRECT && j < g->n_nodes && g->nodes[j].op == SAM3_OP_GELU &&
	    g->nodes[j].n_inputs >= 1 && g->nodes[j].inputs[0] == out && uses_of(uses, out) == 1 &&
	    g->nodes[j].output && s3h_nelems(g->nodes[j].output) == ny) {
		out = g->nodes[j].output;
		flags |= S3K_EPI_GELU;
		j++;
	}
	void *dbias = NULL;
	if (bias)
		err = dev_in(hb, bias, &dbias);
	if (err == SAM3_OK)
		err = dev_out(hb, out, &ty.data);
	if (err != SAM3_OK)
		return err;
	err = transposed ? s3h_conv_transpose2d(&dn, dbias, flags, path, hb->stream)
			 : s3h_conv2d(&dn, dbias, flags, path, hb->stream);
	if (err == SAM3_OK) {
		hb->stats.gpu_nodes++;
		hb->stats.fused_nodes += j - i - 1;
		*used = j - i;
	}
	return err;
}

/* ADD, GELU, TRANSPOSE, SDPA, LAYERNORM, ROPE, SLICE on device copies of
 * the node's tensors. */
static enum sam3_error run_elementwise(struct sam3_hip_backend *hb, const struct sam3_node *n)
{
	struct sam3_tensor tin[SAM3_NODE_MAX_INPUTS], tout;
	struct sam3_node dn = *n;
	enum sam3_error err = SAM3_OK;
	for (int k = 0; k < n->n_inputs && k < SAM3_NODE_MAX_INPUTS; k++) {
		if (!n->inputs[k])
			continue;
		tin[k] = *n->inputs[k];
		err = dev_in(hb, n->inputs[k], &tin[k].data);
		if (err != SAM3_OK)
			return err;
		dn.inputs[k] = &tin[k];
	}
	if (!n->output) {
		s3h_error("graph_eval: NULL output");
		return SAM3_EINVAL;
	}
	tout = *n->output;
	err = dev_out(hb, n->output, &tout.data);
	if (err != SAM3_OK)
		return err;
	dn.output = &tout;
	if (n->op == SAM3_OP_ADD)
		err = s3h_add(&dn, hb->stream);
	else if (n->op == SAM3_OP_GELU)
		err = s3h_gelu(&dn, hb->stream);
	else if (n->op == SAM3_OP_SDPA)
		err = sam3_hip_kernel_sdpa(&dn, hb->stream);
	else if (n->op == SAM3_OP_LAYERNORM)
		err = s3h_layernorm(&dn, hb->stream);
	else if (n->op == SAM3_OP_ROPE)
		err = s3h_rope(&dn, hb->stream);
	else if (n->op == SAM3_OP_SLICE)
		err = s3h_slice(&dn, hb->stream);
	else if (n->op == SAM3_OP_BIAS_ADD)
		err = s3h_bias_add(&dn, hb->stream);
	else if (n->op == SAM3_OP_MAXPOOL2D)
		err = s3h_maxpool2d(&dn, hb->stream);
	else if (n->op == SAM3_OP_CAST)
		err = sam3_hip_kernel_cast(&dn, hb->stream);
	else
		err = s3h_transpose(&dn, hb->stream);
	if (err == SAM3_OK)
		hb->stats.gpu_nodes++;
	return err;
}

/* gh_multihead_attention_rope's head merge (graph_helpers.c:721-882):
 * an SDPA node whose one reader is TRANSPOSE (0,2,1,3) of its
 * [B, H, Sq, D] output: the attention kernel stores the merged rows
 * itself, as f32 or, when a GEMM reads them as its A (rows of H*D), in
 * that GEMM's operand form (*fmt; f32 SDPA with head size 64). Returns
 * the transpose's node index, or -1. Storing the transpose's output at
 * node i must change nothing another node before it reads or writes. */
static int sdpa_merge_target(struct sam3_hip_backend *hb, const struct sam3_graph *g, int i,
			     struct use_map *uses, const unsigned char *done, int *fmt)
{
	const struct s3h_settings *set = s3h_settings();
	const struct sam3_node *n = &g->nodes[i];
	if (!set->sdpa_merge || n->op != SAM3_OP_SDPA || !n->output || !s3h_sdpa_node_ok(n))
		return -1;
	const struct sam3_tensor *o = n->output, *q = n->inputs[0];
	if (q->n_dims != 4 || o->n_dims != 4 || !dims_are(o, q->dims[0], q->dims[1], q->dims[2],
							   n->params[0]) ||
	    uses_of(uses, o) != 1)
		return -1;
	const int j = next_reader(g, i + 1, o);
	if (j < 0 || done[j])
		return -1;
	const struct sam3_node *t = &g->nodes[j];
	if (t->op != SAM3_OP_TRANSPOSE || t->n_inputs < 1 || t->inputs[0] != o || !t->output ||
	    t->params[0] != 0 || t->params[1] != 2 || t->params[2] != 1 || t->params[3] != 3 ||
	    t->output->dtype != o->dtype ||
	    !dims_are(t->output, o->dims[0], o->dims[2], o->dims[1], o->dims[3]))
		return -1;
	int k = 0;
	*fmt = set->permute_operand ? permute_operand_form(hb, g, j, uses, &k) : S3H_A_PLAIN;
	if (*fmt != S3H_A_PLAIN &&
	    (o->dtype != SAM3_DTYPE_F32 || n->params[0] != 64 || k != o->dims[1] * o->dims[3]))
		return -1;
	for (int m = i + 1; m < j; m++) {
		const struct sam3_node *x = &g->nodes[m];
		if (same_data(x->output, t->output))
			return -1;
		for (int r = 0; r < x->n_inputs && r < SAM3_NODE_MAX_INPUTS; r++)
			if (same_data(x->inputs[r], t->output))
				return -1;
	}
	return j;
}

static enum sam3_error run_sdpa_merged(struct sam3_hip_backend *hb, const struct sam3_node *n,
				       const struct sam3_node *t, int fmt)
{
	struct sam3_tensor tin[SAM3_NODE_MAX_INPUTS];
	struct sam3_node dn = *n;
	enum sam3_error err = SAM3_OK;
	for (int k = 0; k < n->n_inputs && k < SAM3_NODE_MAX_INPUTS; k++) {
		if (!n->inputs[k])
			continue;
		tin[k] = *n->inputs[k];
		err = dev_in(hb, n->inputs[k], &tin[k].data);
		if (err != SAM3_OK)
			return err;
		dn.inputs[k] = &tin[k];
	}
	if (fmt != S3H_A_PLAIN) {
		int BH = 0, Sq = 0, Sk = 0;
		const struct sam3_tensor *q = dn.inputs[0];
		if (q->n_dims == 4) {
			BH = q->dims[0] * q->dims[1];
			Sq = q->dims[2];
			Sk = dn.inputs[1]->dims[2];
		}
		/* the operand forms are written by the MFMA kernel only: any
		 * other case runs the two nodes as they are */
		if (s3k_attn_path(q->dtype, q->data, dn.inputs[1]->data, dn.inputs[2]->data, q->data, BH,
				  Sq, Sk, n->params[0]) != S3K_ATTN_MFMA) {
			err = run_elementwise(hb, n);
			if (err == SAM3_OK)
				err = run_permute_as(hb, t, fmt, q->dims[1] * n->params[0]);
			return err;
		}
	}
	void *dy = NULL;
	if (fmt == S3H_A_PLAIN)
		err = dev_out(hb, t->output, &dy);
	else
		err = dev_out_fmt(hb, t->output,
				  (size_t)s3h_nelems(t->output) * (fmt == S3H_A_PLANES ? 6 : 2), fmt, &dy,
				  NULL);
	if (err == SAM3_OK)
		err = s3h_sdpa_merged(&dn, dy, fmt, hb->ovf, hb->ovf_tag, hb->stream);
	if (err == SAM3_OK) {
		hb->stats.gpu_nodes++;
		hb->stats.fused_nodes++;
		if (fmt != S3H_A_PLAIN) {
			hb->stats.operand_writes++;
			hb->f16_writes += fmt == S3H_A_F16;
		}
	}
	return err;
}

static int runs_on_gpu(const struct sam3_node *n)
{
	if (n->n_inputs < 1 || !n->inputs[0])
		return 0;
	if (n->op == SAM3_OP_SDPA)
		return s3h_sdpa_node_ok(n);
	if (n->op == SAM3_OP_ROPE)
		return s3h_rope_ok(n);
	const int dt = n->inputs[0]->dtype;
	for (int k = 1; k < n->n_inputs; k++)
		if (n->inputs[k] && (int)n->inputs[k]->dtype != dt)
			return 0;
	switch (n->op) {
	case SAM3_OP_ADD:
	case SAM3_OP_GELU:
		return float_dt(dt);
	case SAM3_OP_BIAS_ADD:
		return s3h_bias_add_ok(n);
	case SAM3_OP_MAXPOOL2D:
		return s3h_maxpool2d_ok(n);
	case SAM3_OP_TRANSPOSE:
		return s3h_transpose_ok(n);
	case SAM3_OP_LAYERNORM:
		return s3h_layernorm_ok(n);
	case SAM3_OP_SLICE:
		return s3h_slice_ok(n);
	case SAM3_OP_CAST:
		return s3h_cast_ok(n);
	default:
		return 0;
	}
}

static enum sam3_error run_host(struct sam3_hip_backend *hb, const struct sam3_node *n)
{
	if (!hb->host_fn) {
		s3h_error("graph_eval: no HIP kernel for op=%d and no host dispatcher", n->op);
		return SAM3_EDTYPE;
	}
	enum sam3_error err = SAM3_OK;
	for (int k = 0; k < n->n_inputs && k < SAM3_NODE_MAX_INPUTS; k++) {
		if (!n->inputs[k] || !n->inputs[k]->data)
			continue;
		struct s3h_res *e = res_find(hb, n->inputs[k]->data);
		if (e && e->dev_valid && !e->host_valid)
			err = download(hb, e);
		if (err != SAM3_OK)
			return err;
	}
	err = s3h_hip(hipStreamSynchronize(hb->stream), "graph_eval: sync before host op");
	if (err != SAM3_OK)
		return err;
	err = hb->host_fn(n, hb->host_ctx);
	if (err != SAM3_OK)
		return err;
	if (n->output && n->output->data) {
		struct s3h_res *e = res_find(hb, n->output->data);
		if (e) {
			e->dev_valid = 0;
			e->host_valid = 1;
			e->produced = 0;
		}
	}
	hb->stats.host_nodes++;
	return SAM3_OK;
}

/* The nodes of g in order, as cpu_graph_eval runs them
 * (cpu_backend.c:134-148), with this backend's folds. */
static enum sam3_error run_nodes(struct sam3_hip_backend *hb, const struct sam3_graph *g,
				 struct use_map *uses_p, unsigned char *folded, unsigned char *done)
{
	enum sam3_error err = SAM3_OK;
	struct use_map uses = *uses_p;
	const struct s3h_settings *set = s3h_settings();
	const int qkv_plain = !set->qkv_chain;
	const int ln_plain = !set->ln_operand;
	const int perm_plain = !set->permute_operand;
	int ln_fmt = S3H_A_PLAIN, perm_k = 0, merge_j = -1, merge_fmt = S3H_A_PLAIN;
	const int part_plain = !set->partition_fold;
	int lrm[3] = {0, 0, 0}, lchain[8], lnc = 0;
	const struct sam3_tensor *lt = NULL;
	struct s3h_ln_in lng;
	struct s3h_att1_in att1;

	for (int i = 0; i < g->n_nodes && err == SAM3_OK;) {
		const struct sam3_node *n = &g->nodes[i];
		int used = 1;
		struct qkv_chain qc;
		if (n->op == SAM3_OP_NONE || done[i]) {
			err = SAM3_OK; /* done[i]: run earlier as part of a chain */
		} else if (n->op == SAM3_OP_SLICE && !qkv_plain && match_qkv_chain(g, i, &uses, &qc)) {
			err = run_qkv_chains(hb, g, &qc, &uses, done);
		} else if (n->op == SAM3_OP_RESHAPE) {
			/* a view: consumers find the input's device copy under the
			 * same host address */
			err = s3h_reshape(n);
		} else if (n->op == SAM3_OP_TRANSPOSE && transpose_folds(g, i, &uses)) {
			folded[i] = 1;
			hb->stats.fused_nodes++;
		} else if (n->op == SAM3_OP_MATMUL) {
			err = run_matmul(hb, g, i, folded, done, &uses, &used);
		} else if ((n->op == SAM3_OP_CONV2D && s3h_conv2d_ok(n)) ||
			   (n->op == SAM3_OP_CONV_TRANSPOSE2D && s3h_conv_transpose2d_ok(n))) {
			err = run_conv(hb, g, i, &uses, &used);
		} else if (n->op == SAM3_OP_LAYERNORM && ln_gemv_form(hb, g, i, &uses, &lng)) {
			err = run_layernorm_gemv(hb, n, &lng);
		} else if (n->op == SAM3_OP_LAYERNORM && !ln_plain && !part_plain &&
			   (ln_fmt = ln_partition_form(hb, g, i, &uses, lrm, lchain, &lnc, &lt)) !=
				   S3H_A_PLAIN) {
			err = run_layernorm_map(hb, n, ln_fmt, lrm, lt);
			if (err == SAM3_OK) {
				for (int k = 0; k < lnc; k++)
					done[lchain[k]] = 1;
				hb->stats.fused_nodes += lnc;
			}
		} else if (n->op == SAM3_OP_LAYERNORM && !ln_plain &&
			   (ln_fmt = ln_operand_form(hb, g, i, &uses)) != S3H_A_PLAIN) {
			err = run_layernorm_as(hb, n, ln_fmt);
		} else if (n->op == SAM3_OP_TRANSPOSE && !perm_plain &&
			   (ln_fmt = permute_operand_form(hb, g, i, &uses, &perm_k)) != S3H_A_PLAIN) {
			err = run_permute_as(hb, n, ln_fmt, perm_k);
		} else if (n->op == SAM3_OP_SDPA &&
			   (merge_j = sdpa_gemv_form(hb, g, i, &uses, done, &att1)) >= 0) {
			err = run_sdpa_gemv(hb, &g->nodes[merge_j], &att1);
			if (err == SAM3_OK)
				done[merge_j] = 1;
		} else if (n->op == SAM3_OP_SDPA &&
			   (merge_j = sdpa_merge_target(hb, g, i, &uses, done, &merge_fmt)) >= 0) {
			err = run_sdpa_merged(hb, n, &g->nodes[merge_j], merge_fmt);
			if (err == SAM3_OK)
				done[merge_j] = 1;
		} else if (runs_on_gpu(n)) {
			err = run_elementwise(hb, n);
		} else {
			err = run_host(hb, n);
		}
		if (err != SAM3_OK)
			s3h_error("hip_graph_eval: node %d (op=%d) failed", i, n->op);
		i += used;
	}

	return err;
}

static enum sam3_error hip_graph_eval(struct sam3_backend *be, struct sam3_graph *g)
{
	struct sam3_hip_backend *hb = (struct sam3_hip_backend *)be;
	enum sam3_error err;

	if (!be || !g) {
		s3h_error("graph_eval: NULL argument");
		return SAM3_EINVAL;
	}
	memset(&hb->stats, 0, sizeof(hb->stats));
	if (g->n_nodes <= 0)
		return SAM3_OK;
	err = s3h_hip(hipSetDevice(hb->device), "graph_eval: set device");
	if (err != SAM3_OK)
		return err;

	struct use_map uses;
	err = build_uses(g, &uses);
	if (err != SAM3_OK)
		return err;
	unsigned char *folded = calloc((size_t)g->n_nodes, 1);
	unsigned char *done = calloc((size_t)g->n_nodes, 1);
	if (!folded || !done) {
		free(folded);
		free(done);
		free(uses.key);
		free(uses.count);
		s3h_error("graph_eval: out of host memory");
		return SAM3_ENOMEM;
	}
	for (int i = 0; i < hb->n_res; i++)
		hb->res[i].produced = hb->res[i].fresh = 0;
	s3h_cur = hb;
	hb->no_f16_ops = 0;
	hb->f16_writes = 0;
	hb->n_rowf = 0;
	hb->ovf_tag = hb->ovf_tag + 1 ? hb->ovf_tag + 1 : 1;
	err = run_nodes(hb, g, &uses, folded, done);
	if (err == SAM3_OK)
		err = rowf_flush(hb);
	hb->n_rowf = 0;
	/* A fused producer that wrote an f16 GEMM operand flags values the
	 * f16 copy cannot hold (|x| >= 2^15, or rows of tiny values: per row
	 * for LayerNorm and the GEMM epilogue, per four values for the
	 * permute and the attention kernel's merged heads). Then
	 * the graph runs again without f16 operand forms: the consumers read
	 * f32 and make their row-scaled f16 copy themselves. The graph's
	 * inputs are unchanged by the first run (nodes write only their own
	 * outputs), so the second run starts from the same state. */
	if (err == SAM3_OK && hb->f16_writes) {
		unsigned tag = 0;
		err = s3h_hip(hipMemcpyAsync(&tag, hb->ovf, sizeof(tag), hipMemcpyDeviceToHost,
					     hb->stream),
			      "graph_eval: range flag");
		if (err == SAM3_OK)
			err = s3h_hip(hipStreamSynchronize(hb->stream), "graph_eval: range flag");
		if (err == SAM3_OK && tag == hb->ovf_tag) {
			const struct sam3_hip_eval_stats first = hb->stats;
			memset(&hb->stats, 0, sizeof(hb->stats));
			hb->stats.range_reruns = first.range_reruns + 1;
			memset(folded, 0, (size_t)g->n_nodes);
			memset(done, 0, (size_t)g->n_nodes);
			hb->no_f16_ops = 1;
			err = run_nodes(hb, g, &uses, folded, done);
			hb->no_f16_ops = 0;
		}
	}

	/* Readback of the graph's final outputs: node outputs no node of the
	 * graph consumes, as the reference's GPU backend does
	 * (metal_backend.c:1805-1850, 1897-1945). Intermediates stay on the
	 * device. SAM3_HIP_READBACK=all downloads every produced tensor. */
	if (err == SAM3_OK && !g->no_readback) {
		if (s3h_settings()->readback_all) {
			for (int i = 0; i < hb->n_res && err == SAM3_OK; i++) {
				struct s3h_res *e = &hb->res[i];
				if (e->produced && e->dev_valid && !e->host_valid && !e->fmt)
					err = download(hb, e);
			}
		} else {
			for (int i = 0; i < g->n_nodes && err == SAM3_OK; i++) {
				const struct sam3_tensor *t = g->nodes[i].output;
				if (!t || !t->data || uses_of(&uses, t) > 0)
					continue;
				struct s3h_res *e = res_find(hb, t->data);
				if (e && e->produced && e->dev_valid && !e->host_valid && !e->fmt)
					err = download(hb, e);
			}
		}
	}
	enum sam3_error serr = s3h_hip(hipStreamSynchronize(hb->stream), "graph_eval: sync");
	if (err == SAM3_OK)
		err = serr;
	s3h_cur = NULL;
	/* Intermediates' contents end with the eval; final outputs stay
	 * resident and valid, so a later graph reads them without a copy (the
	 * reference's GPU backend evicts and keeps the same sets,
	 * metal_backend.c:1897-1908). An intermediate keeps its allocation
	 * for the next eval that produces the same host tensor, but is marked
	 * stale: read as an input later, it is uploaded from the host. A view
	 * of an intermediate that is a final output keeps the shared copy. */
	for (int i = 0; i < g->n_nodes; i++) {
		const struct sam3_tensor *t = g->nodes[i].output;
		struct s3h_res *e = t && t->data && uses_of(&uses, t) > 0 ? res_find(hb, t->data) : NULL;
		if (e && e->produced) {
			e->dev_valid = 0;
			e->fmt = 0;
			e->keep = 1;
		}
	}
	for (int i = 0; i < g->n_nodes; i++) {
		const struct sam3_tensor *t = g->nodes[i].output;
		struct s3h_res *e = t && t->data && uses_of(&uses, t) == 0 ? res_find(hb, t->data) : NULL;
		if (e && e->produced)
			e->dev_valid = 1;
	}
	for (int i = hb->n_res - 1; i >= 0; i--)
		if (!hb->res[i].keep)
			res_drop_at(hb, i);
	free(folded);
	free(done);
	free(uses.key);
	free(uses.count);
	return err;
}

/* ------------------------------------------------------------------ */
/* vtable                                                               */
/* ------------------------------------------------------------------ */
static enum sam3_error hip_init(struct sam3_backend *be)
{
	struct sam3_hip_backend *hb = (struct sam3_hip_backend *)be;
	int n = 0;
	if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
		(void)hipGetLastError();
		s3h_error("hip backend: no HIP device");
		return SAM3_EBACKEND;
	}
	if (hb->device < 0 || hb->device >= n) {
		s3h_error("hip backend: device %d out of range (%d devices)", hb->device, n);
		return SAM3_EINVAL;
	}
	enum sam3_error err = s3h_hip(hipSetDevice(hb->device), "hip backend: set device");
	if (err == SAM3_OK)
		err = s3h_hip(hipStreamCreateWithFlags(&hb->stream, hipStreamNonBlocking),
			      "hip backend: stream");
	if (err == SAM3_OK)
		err = s3h_hip(hipMalloc((void **)&hb->ovf, 256), "hip backend: range flag");
	if (err == SAM3_OK)
		err = s3h_hip(hipMemset(hb->ovf, 0, 256), "hip backend: range flag");
	return err;
}

static void hip_free(struct sam3_backend *be)
{
	struct sam3_hip_backend *hb = (struct sam3_hip_backend *)be;
	if (!hb)
		return;
	(void)hipSetDevice(hb->device);
	while (hb->n_res)
		res_drop_at(hb, hb->n_res - 1);
	free(hb->res);
	hb->res = NULL;
	hb->cap_res = 0;
	free(hb->res_ix);
	hb->res_ix = NULL;
	hb->res_ix_cap = 0;
	while (hb->n_blobs)
		blob_drop_at(hb, hb->n_blobs - 1);
	free(hb->blobs);
	hb->blobs = NULL;
	hb->cap_blobs = 0;
	if (hb->stream)
		(void)hipStreamSynchronize(hb->stream);
	for (int i = 0; i < hb->n_owned; i++)
		(void)hipFree(hb->owned[i]);
	free(hb->owned);
	hb->owned = NULL;
	hb->n_owned = hb->cap_owned = 0;
	free(hb->prep);
	hb->prep = NULL;
	hb->n_prep = hb->cap_prep = 0;
	s3h_stager_free(&hb->stager);
	if (hb->stream) {
		s3h_scratch_release(hb->stream);
		(void)hipStreamSynchronize(hb->stream);
		(void)hipStreamDestroy(hb->stream);
		hb->stream = NULL;
	}
	if (hb->arena) {
		(void)hipHostFree(hb->arena);
		hb->arena = NULL;
	}
	if (hb->ovf) {
		(void)hipFree(hb->ovf);
		hb->ovf = NULL;
	}
}

/* Same contract as cpu_alloc_tensor (cpu_backend.c:84-118): n_dims in
 * [1, 4], a dtype with an element size, fills data/nbytes/strides; memory
 * is pinned host memory from the backend's arena. */
static enum sam3_error hip_alloc_tensor(struct sam3_backend *be, struct sam3_tensor *t)
{
	struct sam3_hip_backend *hb = (struct sam3_hip_backend *)be;
	if (!t) {
		s3h_error("HIP alloc_tensor: NULL tensor");
		return SAM3_EINVAL;
	}
	if (t->n_dims < 1 || t->n_dims > SAM3_MAX_DIMS) {
		s3h_error("HIP alloc_tensor: invalid n_dims=%d", t->n_dims);
		return SAM3_EINVAL;
	}
	size_t es = s3h_dtype_size(t->dtype);
	if (es == 0) {
		s3h_error("HIP alloc_tensor: unknown dtype=%d", t->dtype);
		return SAM3_EINVAL;
	}
	if (!hb->arena) {
		const int mb = s3h_settings()->arena_mb;
		size_t sz = mb > 0 ? (size_t)mb << 20 : S3H_ARENA_DEFAULT;
		if (!sz)
			sz = S3H_ARENA_DEFAULT;
		enum sam3_error err = s3h_hip(hipHostMalloc((void **)&hb->arena, sz,
							    hipHostMallocDefault),
					      "HIP alloc_tensor: pinned arena");
		if (err != SAM3_OK)
			return err;
		hb->arena_size = sz;
		hb->arena_off = 0;
	}
	size_t nbytes = (size_t)s3h_nelems(t) * es;
	size_t off = (hb->arena_off + S3H_ARENA_ALIGN - 1) & ~(size_t)(S3H_ARENA_ALIGN - 1);
	if (off + nbytes > hb->arena_size) {
		s3h_error("HIP alloc_tensor: OOM (%zu bytes requested, %zu / %zu used)", nbytes,
			  hb->arena_off, hb->arena_size);
		return SAM3_ENOMEM;
	}
	t->data = hb->arena + off;
	hb->arena_off = off + nbytes;
	t->nbytes = nbytes;
	int s = 1;
	for (int i = t->n_dims - 1; i >= 0; i--) {
		t->strides[i] = s;
		s *= t->dims[i];
	}
	return SAM3_OK;
}

static void hip_arena_reset(struct sam3_backend *be)
{
	struct sam3_hip_backend *hb = (struct sam3_hip_backend *)be;
	if (hb->arena)
		res_drop_range(hb, hb->arena, hb->arena + hb->arena_size);
	hb->arena_off = 0;
}

static void hip_cache_invalidate(struct sam3_backend *be, const void *start, size_t len)
{
	struct sam3_hip_backend *hb = (struct sam3_hip_backend *)be;
	const char *lo = (const char *)start, *hi = lo + len;
	res_drop_range(hb, lo, hi);
	for (int i = hb->n_blobs - 1; i >= 0; i--)
		if (hb->blobs[i].host < hi && hb->blobs[i].host + hb->blobs[i].nbytes > lo)
			blob_drop_at(hb, i);
}

static const struct sam3_backend_ops hip_ops = {
	.init             = hip_init,
	.free             = hip_free,
	.alloc_tensor     = hip_alloc_tensor,
	.graph_eval       = hip_graph_eval,
	.arena_reset      = hip_arena_reset,
	.cache_invalidate = hip_cache_invalidate,
};

const struct sam3_backend_ops *sam3_hip_backend_ops(void)
{
	return &hip_ops;
}

struct sam3_backend *sam3_hip_backend_create(int device)
{
	struct sam3_hip_backend *hb = calloc(1, sizeof(*hb));
	if (!hb) {
		s3h_error("hip backend: out of host memory");
		return NULL;
	}
	/* sam3.c's enum has CPU and METAL only; the object is told apart by
	 * its ops table, and `type` stays CPU so model code keeps its
	 * host-memory behaviour (image_encoder.c:703 checks METAL). */
	hb->base.type = SAM3_BACKEND_CPU;
	hb->base.ops = &hip_ops;
	hb->device = device;
	if (hip_ops.init(&hb->base) != SAM3_OK) {
		hip_free(&hb->base);
		free(hb);
		return NULL;
	}
	return &hb->base;
}

void sam3_hip_backend_destroy(struct sam3_backend *be)
{
	if (!be)
		return;
	be->ops->free(be);
	free(be);
}

void sam3_hip_backend_set_host_dispatch(struct sam3_backend *be, sam3_hip_host_dispatch_fn fn,
					void *ctx)
{
	struct sam3_hip_backend *hb = (struct sam3_hip_backend *)be;
	if (!hb)
		return;
	hb->host_fn = fn;
	hb->host_ctx = ctx;
}

void *sam3_hip_backend_stream(struct sam3_backend *be)
{
	return be ? (void *)((struct sam3_hip_backend *)be)->stream : NULL;
}

void sam3_hip_backend_last_stats(struct sam3_backend *be, struct sam3_hip_eval_stats *out)
{
	if (!be || !out)
		return;
	*out = ((struct sam3_hip_backend *)be)->stats;
}

/* ------------------------------------------------------------------ */
/* Weights in HBM                                                       */
/* ------------------------------------------------------------------ */
enum sam3_error sam3_hip_backend_map_weights(struct sam3_backend *be, const void *host,
					     size_t nbytes)
{
	struct sam3_hip_backend *hb = (struct sam3_hip_backend *)be;
	if (!hb || !host || !nbytes) {
		s3h_error("map_weights: NULL backend or empty range");
		return SAM3_EINVAL;
	}
	const char *lo = (const char *)host, *hi = lo + nbytes;
	for (int i = 0; i < hb->n_blobs; i++)
		if (hb->blobs[i].host < hi && hb->blobs[i].host + hb->blobs[i].nbytes > lo) {
			s3h_error("map_weights: range overlaps a mapped range");
			return SAM3_EINVAL;
		}
	if (is_device_ptr(host)) {
		s3h_error("map_weights: range is device memory");
		return SAM3_EINVAL;
	}
	enum sam3_error err = s3h_hip(hipSetDevice(hb->device), "map_weights: set device");
	if (err == SAM3_OK)
		err = s3h_stager_init(&hb->stager, hb->device);
	if (err != SAM3_OK)
		return err;
	if (hb->n_blobs == hb->cap_blobs) {
		int cap = hb->cap_blobs ? hb->cap_blobs * 2 : 4;
		struct s3h_blob *b = realloc(hb->blobs, (size_t)cap * sizeof(*b));
		if (!b) {
			s3h_error("map_weights: out of host memory");
			return SAM3_ENOMEM;
		}
		hb->blobs = b;
		hb->cap_blobs = cap;
	}
	char *dev = NULL;
	err = s3h_hip(hipMalloc((void **)&dev, nbytes), "map_weights: device copy");
	if (err != SAM3_OK)
		return err;
	/* Residency shadows of tensors inside the range become redundant. */
	res_drop_range(hb, lo, hi);
	err = s3h_hip(hipStreamSynchronize(hb->stream), "map_weights: sync");
	if (err == SAM3_OK)
		err = s3h_stager_copy(&hb->stager, dev, host, nbytes);
	if (err != SAM3_OK) {
		(void)hipFree(dev);
		return err;
	}
	hb->blobs[hb->n_blobs++] = (struct s3h_blob){lo, nbytes, dev};
	return SAM3_OK;
}

void *sam3_hip_backend_weight_ptr(struct sam3_backend *be, const void *host)
{
	struct sam3_hip_backend *hb = (struct sam3_hip_backend *)be;
	return hb && host ? blob_addr(hb, host, 1) : NULL;
}

static enum sam3_error own(struct sam3_hip_backend *hb, void *p)
{
	if (hb->n_owned == hb->cap_owned) {
		int cap = hb->cap_owned ? hb->cap_owned * 2 : 16;
		void **o = realloc(hb->owned, (size_t)cap * sizeof(*o));
		if (!o) {
			s3h_error("fuse_rows: out of host memory");
			return SAM3_ENOMEM;
		}
		hb->owned = o;
		hb->cap_owned = cap;
	}
	hb->owned[hb->n_owned++] = p;
	return SAM3_OK;
}

/* Stack parts [d_i, cols] (or [d_i]) of one dtype into one [sum d_i, cols]
 * tensor in HBM. The replacement of image_encoder.c:223-254 (fuse_3),
 * which declares its output F32 whatever the parts are, so Q8_0 parts
 * come out as F32-labelled block bytes. Here the output keeps the parts'
 * dtype. Q8_0 blocks run along the flat index, so a part whose element
 * count is a multiple of 32 is a whole number of blocks and the fused
 * tensor is the byte concatenation; other counts would put one block
 * across two parts and are rejected. */
enum sam3_error sam3_hip_backend_fuse_rows(struct sam3_backend *be,
					   const struct sam3_tensor *const *parts, int n_parts,
					   struct sam3_tensor *out)
{
	struct sam3_hip_backend *hb = (struct sam3_hip_backend *)be;
	if (!hb || !parts || !out || n_parts < 1 || n_parts > SAM3_NODE_MAX_INPUTS) {
		s3h_error("fuse_rows: NULL argument or part count outside [1, %d]",
			  SAM3_NODE_MAX_INPUTS);
		return SAM3_EINVAL;
	}
	const struct sam3_tensor *p0 = parts[0];
	if (!p0 || !p0->data || p0->n_dims < 1 || p0->n_dims > 2) {
		s3h_error("fuse_rows: part 0 must be a 1-D or 2-D tensor with data");
		return SAM3_EINVAL;
	}
	const int dt = p0->dtype, nd = p0->n_dims;
	if (dt != SAM3_DTYPE_Q8_0 && s3h_dtype_size(dt) == 0) {
		s3h_error("fuse_rows: dtype %d has no layout", dt);
		return SAM3_EDTYPE;
	}
	long long rows = 0;
	size_t total = 0;
	for (int i = 0; i < n_parts; i++) {
		const struct sam3_tensor *t = parts[i];
		if (!t || !t->data || t->n_dims != nd || (nd == 2 && t->dims[1] != p0->dims[1]) ||
		    t->dims[0] <= 0 || (nd == 2 && t->dims[1] <= 0)) {
			s3h_error("fuse_rows: part %d does not match part 0's rank and columns", i);
			return SAM3_EINVAL;
		}
		if ((int)t->dtype != dt) {
			s3h_error("fuse_rows: part %d has dtype %d, part 0 has %d", i, t->dtype, dt);
			return SAM3_EDTYPE;
		}
		if (dt == SAM3_DTYPE_Q8_0 && s3h_nelems(t) % 32 != 0) {
			s3h_error("fuse_rows: Q8_0 part %d has %lld elements, not a whole number "
				  "of 32-element blocks", i, s3h_nelems(t));
			return SAM3_EINVAL;
		}
		rows += t->dims[0];
		total += s3h_tensor_bytes(t);
	}
	if (rows > INT32_MAX) {
		s3h_error("fuse_rows: %lld rows", rows);
		return SAM3_EINVAL;
	}
	enum sam3_error err = s3h_hip(hipSetDevice(hb->device), "fuse_rows: set device");
	char *dev = NULL;
	if (err == SAM3_OK)
		err = s3h_hip(hipMalloc((void **)&dev, total), "fuse_rows: device buffer");
	if (err != SAM3_OK)
		return err;
	size_t off = 0;
	for (int i = 0; i < n_parts && err == SAM3_OK; i++) {
		const struct sam3_tensor *t = parts[i];
		const size_t nb = s3h_tensor_bytes(t);
		const void *src = blob_addr(hb, t->data, nb);
		hipMemcpyKind kind = hipMemcpyDeviceToDevice;
		if (!src) {
			src = t->data;
			kind = is_device_ptr(src) ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
		}
		err = s3h_hip(hipMemcpyAsync(dev + off, src, nb, kind, hb->stream), "fuse_rows: copy");
		off += nb;
	}
	if (err == SAM3_OK)
		err = s3h_hip(hipStreamSynchronize(hb->stream), "fuse_rows: sync");
	if (err == SAM3_OK)
		err = own(hb, dev);
	if (err != SAM3_OK) {
		(void)hipStreamSynchronize(hb->stream);
		(void)hipFree(dev);
		return err;
	}
	memset(out, 0, sizeof(*out));
	out->dtype = (enum sam3_dtype)dt;
	out->n_dims = nd;
	out->dims[0] = (int)rows;
	if (nd == 2)
		out->dims[1] = p0->dims[1];
	if (dt != SAM3_DTYPE_Q8_0) {
		int st = 1;
		for (int d = nd - 1; d >= 0; d--) {
			out->strides[d] = st;
			st *= out->dims[d];
		}
	}
	out->data = dev;
	out->nbytes = total;
	return SAM3_OK;
}

/* ------------------------------------------------------------------ */
/* Prepared weights                                                     */
/* ------------------------------------------------------------------ */
void *s3h_prep_find(const void *src, int tag, int rows, int k)
{
	struct sam3_hip_backend *hb = s3h_cur;
	if (!hb)
		return NULL;
	for (int i = 0; i < hb->n_prep; i++) {
		const struct s3h_prep *p = &hb->prep[i];
		if (p->src == (const char *)src && p->tag == tag && p->rows == rows && p->k == k) {
			hb->stats.prep_hits++;
			return p->dev;
		}
	}
	return NULL;
}

int s3h_prep_cacheable(const void *src, size_t src_bytes)
{
	const struct sam3_hip_backend *hb = s3h_cur;
	const char *c = (const char *)src;
	if (!hb || !c)
		return 0;
	for (int i = 0; i < hb->n_blobs; i++) {
		const struct s3h_blob *b = &hb->blobs[i];
		if (c >= b->dev && c < b->dev + b->nbytes && src_bytes <= b->nbytes - (size_t)(c - b->dev))
			return 1;
	}
	for (int i = 0; i < hb->n_res; i++) {
		const struct s3h_res *e = &hb->res[i];
		const char *d = (const char *)e->dev;
		if (d && c >= d && c < d + e->cap && src_bytes <= e->cap - (size_t)(c - d))
			return e->keep && !e->written && e->dev_valid;
	}
	/* a prepared copy is itself constant */
	for (int i = 0; i < hb->n_prep; i++) {
		const char *d = (const char *)hb->prep[i].dev;
		if (c >= d && c < d + hb->prep[i].bytes && src_bytes <= hb->prep[i].bytes - (size_t)(c - d))
			return 1;
	}
	return 0;
}

enum sam3_error s3h_prep_store(const void *src, int tag, int rows, int k, void *dev, size_t bytes)
{
	struct sam3_hip_backend *hb = s3h_cur;
	if (!hb) {
		s3h_error("prepared weight: no graph_eval running");
		return SAM3_EINVAL;
	}
	if (hb->n_prep == hb->cap_prep) {
		int cap = hb->cap_prep ? hb->cap_prep * 2 : 32;
		struct s3h_prep *p = realloc(hb->prep, (size_t)cap * sizeof(*p));
		if (!p) {
			s3h_error("prepared weight: out of host memory");
			return SAM3_ENOMEM;
		}
		hb->prep = p;
		hb->cap_prep = cap;
	}
	hb->prep[hb->n_prep++] = (struct s3h_prep){(const char *)src, tag, rows, k, dev, bytes};
	return SAM3_OK;
}
